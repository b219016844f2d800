// jy_layout.h — the HBM layout of Q8_0 weight matrices (device-side accessors).
//
// A matrix of N rows x K cols (nb = K/32 blocks of 32 weights, one fp16 scale
// each) is stored as row groups of 4 rows x chunks of 8 blocks:
//   nch = ceil(nb/8) chunks, nbp = 8*nch, rows padded to a multiple of 4, nchp >= nch
//   chunks stored per row group (zero chunks after the real ones);
//   qs : 1 KiB per (row group rg, chunk ch) at qs + (rg*nchp + ch)*1024.  Inside it,
//        thread slot t = r*16 + g (r = row in group, g = lane pair 0..15) owns 16
//        bytes: for block j = 0..7 of the chunk, bytes 2j, 2j+1 = weights of
//        lanes 2g, 2g+1.  A wave (64 lanes x 16 B) therefore reads 1 KiB
//        contiguous per chunk and each lane gets the two lanes it accumulates.
//   d  : 64 B per (rg, ch) at d + (rg*nchp + ch)*32 halves; row r's eight block
//        scales at [r*8 .. r*8+7].
// Padding blocks and rows are zero, so they add exact zeros.  Bytes per 32
// weights stay 34, only the order changes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jieyu_model.h"
#include "jy_device.h"
#include "jy_kernels.h"

namespace jy {

__device__ __forceinline__ size_t q8_chunk(const Q8Dev& W, int R, int ch) {
    return (size_t)(R >> 2) * W.nchp + ch;
}

// weight (row R, column k) as the exact float q*d
__device__ __forceinline__ float q8_elem(const Q8Dev& W, int R, int k) {
    const int b = k >> 5, L = k & 31, g = L >> 1, c = L & 1, ch = b >> 3, j = b & 7, ri = R & 3;
    const size_t chunk = q8_chunk(W, R, ch);
    const int8_t q = (int8_t)W.qs[chunk * 1024 + (size_t)(ri * 16 + g) * 16 + j * 2 + c];
    return (float)q * half_to_float(W.d[chunk * 32 + ri * 8 + j]);
}

// ---- k-quants (KQDev in jy_kernels.h)
//
// Weight values (libs/matmul_libs/matmul_q.h:47-100, libs/file_libs/q4/q4.h:8-35):
//   Q4_K / Q5_K: fma(q, d*sc, -(dmin*m)) with the 6-bit (sc, m) of 32-weight step c
//                (get_scale_min_k4, matmul_q.h:22-33) and q the nibble (+16 * the
//                fifth bit for Q5_K).  d*sc, dmin*m and q*(d*sc) are exact in float
//                (<= 22 significant bits), so this is the reference's one rounding of
//                d1*q - n1 whether or not it is fused.
//   Q6_K:        (d * sc) * (q - 32) with the int8 scale of each 16 weights: exact.

// weight (row R, column k) of a repacked k-quant matrix
__device__ __forceinline__ float kq_elem(const KQDev& W, int R, int k) {
    const int sb = k >> 8, e = k & 255, c = e >> 5, L = e & 31, g = L >> 1, u = L & 1, ri = R & 3;
    const int T = 2 * (c >> 2) + u, kb = c & 3;
    const size_t chunk = (size_t)(R >> 2) * W.nsb + sb;
    const int t = ri * 16 + g;
    const uint8_t nb = W.nib[(chunk * 64 + t) * 8 + c];
    int q = u ? (nb >> 4) : (nb & 15);
    const uint8_t* h = W.hdr + chunk * 64 + ri * 16;
    const uint32_t dm = W.dm[chunk * 4 + ri];
    const float d = half_to_float((uint16_t)(dm & 0xffffu));
    if (W.type == JY_Q6_K) {
        const uint32_t hb = *reinterpret_cast<const uint32_t*>(W.hi + (chunk * 64 + t) * 4);
        q = (q | (int)(((hb >> (8 * kb + 2 * T)) & 3u) << 4)) - 32;
        const int8_t sc = (int8_t)h[(g >> 3) * 8 + c];
        return (d * (float)sc) * (float)q;
    }
    if (W.type == JY_Q5_K) {
        const uint16_t hb = *reinterpret_cast<const uint16_t*>(W.hi + (chunk * 64 + t) * 2);
        q += ((hb >> (4 * T + kb)) & 1) << 4;
    }
    const float dmin = half_to_float((uint16_t)(dm >> 16));
    return __builtin_fmaf((float)q, d * (float)h[c], -(dmin * (float)h[8 + c]));
}

// RMSNorm of one row already staged in LDS, by the whole workgroup, written to y
// (libs/model_libs/rmsnorm/x86/x86_classic.txt:2-26; eps 1e-5): 16 FMA lanes over
// x^2 (lane l takes elements 16c+l; an 8-wide remainder pass feeds lanes 0..7),
// ((v0+v1) -> halves -> two hadds), then the scalar tail of t < 8 elements as GCC
// builds it (with t >= 4 the first four squares are rounded products added in
// order, the rest fused), den = ss/n + eps, scale = 1/sqrtf(den),
// y = (x*scale)*w.  red: 18 floats of shared memory.
// The scale part: red[16] = 1/sqrtf(den), red[17] = 1 where den <= 0 (the row then
// normalises to zeros); both visible to the whole workgroup on return.
__device__ __forceinline__ void block_rms_scale(const float* x, int n, float* red) {
    const int t = threadIdx.x;
    const int n16 = n / 16 * 16;
    const bool rem8 = n16 + 8 <= n;
    if (t < 16) {
        float a = 0.0f;
#pragma unroll 8
        for (int i = t; i < n16; i += 16) a = __builtin_fmaf(x[i], x[i], a);
        if (t < 8 && rem8) a = __builtin_fmaf(x[n16 + t], x[n16 + t], a);
        red[t] = a;
    }
    __syncthreads();
    if (t == 0) {
        float s[8], q[4];
#pragma unroll
        for (int l = 0; l < 8; l++) s[l] = red[l] + red[8 + l];
#pragma unroll
        for (int l = 0; l < 4; l++) q[l] = s[l] + s[4 + l];
        float ss = (q[0] + q[1]) + (q[2] + q[3]);
        int i = n16 + (rem8 ? 8 : 0);
        if (n - i >= 4)
            for (const int e = i + 4; i < e; i++) ss = ss + x[i] * x[i];
        for (; i < n; i++) ss = __builtin_fmaf(x[i], x[i], ss);
        const float den = ss / (float)n + 1e-5f;
        red[17] = den <= 0.0f ? 1.0f : 0.0f;
        red[16] = den <= 0.0f ? 0.0f : 1.0f / sqrtf(den);
    }
    __syncthreads();
}

__device__ __forceinline__ void block_rmsnorm(const float* x, int n, const float* __restrict__ w,
                                              float* __restrict__ y, float* red) {
    const int t = threadIdx.x;
    block_rms_scale(x, n, red);
    const float scale = red[16];
    const bool zero = red[17] != 0.0f;
    for (int i = t; i < n; i += blockDim.x) y[i] = zero ? 0.0f : (x[i] * scale) * w[i];
}

}  // namespace jy
