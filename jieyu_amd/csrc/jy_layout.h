// jy_layout.h — the HBM layout of Q8_0 weight matrices (device-side accessors).
//
// A matrix of N rows x K cols (nb = K/32 blocks of 32 weights, one fp16 scale
// each) is stored as row groups of 4 rows x chunks of 8 blocks:
//   nch = ceil(nb/8) chunks, nbp = 8*nch, rows padded to a multiple of 4;
//   qs : 1 KiB per (row group rg, chunk ch) at qs + (rg*nch + ch)*1024.  Inside it,
//        thread slot t = r*16 + g (r = row in group, g = lane pair 0..15) owns 16
//        bytes: for block j = 0..7 of the chunk, bytes 2j, 2j+1 = weights of
//        lanes 2g, 2g+1.  A wave (64 lanes x 16 B) therefore reads 1 KiB
//        contiguous per chunk and each lane gets the two lanes it accumulates.
//   d  : 64 B per (rg, ch) at d + (rg*nch + ch)*32 halves; row r's eight block
//        scales at [r*8 .. r*8+7].
// Padding blocks and rows are zero, so they add exact zeros.  Bytes per 32
// weights stay 34, only the order changes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jy_device.h"
#include "jy_kernels.h"

namespace jy {

__device__ __forceinline__ size_t q8_chunk(const Q8Dev& W, int R, int ch) {
    return (size_t)(R >> 2) * W.nch + ch;
}

// weight (row R, column k) as the exact float q*d
__device__ __forceinline__ float q8_elem(const Q8Dev& W, int R, int k) {
    const int b = k >> 5, L = k & 31, g = L >> 1, c = L & 1, ch = b >> 3, j = b & 7, ri = R & 3;
    const size_t chunk = q8_chunk(W, R, ch);
    const int8_t q = (int8_t)W.qs[chunk * 1024 + (size_t)(ri * 16 + g) * 16 + j * 2 + c];
    return (float)q * half_to_float(W.d[chunk * 32 + ri * 8 + j]);
}

}  // namespace jy
