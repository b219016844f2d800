// jy_matvec.h — pieces shared by the decode Q8_0 matvec kernels (the exact
// 32-lane form in jy_matvec.hip, the split-dot form in jy_matvec_split.hip):
// the activation vector's LDS layout and the per-row epilogues.
#pragma once

#include "jy_layout.h"

namespace jy {

// the RMSNorm a decode matvec applies to its input: none, the reference's prologue (the
// normalised vector in LDS before the dot), or by linearity (x times the norm weights in
// LDS, each finished dot times 1/sqrt(ss/K + eps): the tolerance mode)
enum { MV_NORM_NONE = 0, MV_NORM_EXACT = 1, MV_NORM_LINEAR = 2 };

// x in LDS, lane-pair major: element k sits at row (k & 31) >> 1 (the lane pair g that
// reads it), column 2*(k >> 5) + (k & 1); XS = 2 * nbp + 4 floats per row
__device__ __forceinline__ int xs_index(int k, int XS) {
    return ((k & 31) >> 1) * XS + 2 * (k >> 5) + (k & 1);
}

// What a decode matvec does with the finished dot y of row `row` of a row group.  Every
// lane of the row's 16-lane group holds y; the lane with g == 0 owns the row (own).
// All lanes must call this together: the gate/up and q/k pairs are exchanged by a shuffle
// with the partner row (lane ^ 16).
//   STORE   out[row] = y
//   BIAS    out[row] = y + aux[row]
//   RESID   out[row] += y                       (transformer_layer.h:74-77, :86-89)
//   SWIGLU  rows 2j, 2j+1 are gate_j, up_j:  out[j] = silu(gate) * up  (ffn.h:13-17)
//   ROPE    q/k rows: (+ bias), then rope_at on the pair (2m, 2m+1) with the reference's
//           store order inside each group of 8 pairs (rope/x86/x86_classic.txt:10-29);
//           v rows stored as they are
//   ARGMAX  out[row] = y, and the first maximum so far into (best_v, best_i)
// With COH the activations are read and written through to the agent-coherent level
// (act_ld / act_st), for a kernel whose workgroups hand them to each other.
// The per-row operands an epilogue reads from memory (the bias; the residual; RoPE's cos
// and sin at the token's position), loaded by mv_preload when the row group's weight stream
// starts, so that the launch's tail waits for no memory round trip after the last chunk.
struct MvPre {
    float bias = 0.0f, resid = 0.0f, c = 0.0f, s = 0.0f;
};

template <int EPI, bool COH = false>
__device__ __forceinline__ MvPre mv_preload(int row, bool own, int r, const MvArgs& a, const float* out) {
    MvPre p;
    if (EPI == EPI_BIAS || EPI == EPI_ROPE) {
        if (a.aux && own) p.bias = a.aux[row];
    }
    if (EPI == EPI_RESID) {
        if (own) p.resid = act_ld<COH>(out + row);
    }
    if (EPI == EPI_ROPE) {
        if (own && !(r & 1) && row < (a.nh + a.nkv) * a.hd) {
            const int hd = a.hd, half = hd >> 1;
            const int m = (row - row / hd * hd) >> 1;
            const int pos = a.state ? a.state[0] - 1 : a.pos0;
            p.c = a.cos_t[(size_t)pos * half + m];
            p.s = a.sin_t[(size_t)pos * half + m];
        }
    }
    return p;
}

// pre: the row's operands from mv_preload, or nullptr to read them here
template <int EPI, bool COH = false>
__device__ __forceinline__ void mv_epilogue(float y, int row, bool own, int r, int rows, const MvArgs& a,
                                            float* __restrict__ out, float& best_v, int& best_i,
                                            const MvPre* pre = nullptr) {
    const MvPre p = pre ? *pre : mv_preload<EPI, COH>(row, own, r, a, out);
    if (EPI == EPI_STORE) {
        if (own) act_st<COH>(out + row, y);
    } else if (EPI == EPI_BIAS) {
        if (own) act_st<COH>(out + row, y + p.bias);
    } else if (EPI == EPI_RESID) {
        if (own) act_st<COH>(out + row, p.resid + y);
    } else if (EPI == EPI_SWIGLU) {
        const float up = __shfl_xor(y, 16);
        if (own && !(r & 1) && row + 1 < rows) act_st<COH>(out + (row >> 1), silu_ref(y) * up);
    } else if (EPI == EPI_ROPE) {
        const float yb = a.aux ? y + (own ? p.bias : 0.0f) : y;
        const float partner = __shfl_xor(yb, 16);
        const int qk_rows = (a.nh + a.nkv) * a.hd;
        if (own) {
            if (row >= qk_rows) {
                act_st<COH>(out + row, yb);
            } else if (!(r & 1)) {
                const int hd = a.hd, half = hd >> 1;
                const int head = row / hd, m = (row - head * hd) >> 1;
                const float c = p.c, s = p.s;
                const float y0 = __builtin_fmaf(yb, c, -(partner * s));
                const float y1 = __builtin_fmaf(yb, s, partner * c);
                int dst = m;
                if (m < half / 8 * 8) {
                    const int o = m & 7;
                    dst = m - o + ((o == 2 || o == 3) ? o + 2 : (o == 4 || o == 5) ? o - 2 : o);
                }
                act_st<COH>(out + head * hd + 2 * dst, y0);
                act_st<COH>(out + head * hd + 2 * dst + 1, y1);
            }
        }
    } else if (EPI == EPI_ARGMAX) {
        if (own) {
            act_st<COH>(out + row, y);
            if (y > best_v || (y == best_v && row < best_i)) {
                best_v = y;
                best_i = row;
            }
        }
    }
}

// ARGMAX: the workgroup's first maximum into the partials (rowv / rowi: one slot per row
// of the workgroup's waves); argmax_finish_kernel scans them after the kernel, whose
// boundary makes them visible device-wide (generate.h:57-60)
__device__ __forceinline__ void mv_argmax_partial(float best_v, int best_i, int g, int r, int wave, int nwv,
                                                  float* rowv, int* rowi, const MvArgs& a) {
    if (g == 0) {
        rowv[wave * 4 + r] = best_v;
        rowi[wave * 4 + r] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = rowv[0];
        int bi = rowi[0];
        for (int i = 1; i < nwv * 4; i++)
            if (rowv[i] > bv || (rowv[i] == bv && rowi[i] < bi)) {
                bv = rowv[i];
                bi = rowi[i];
            }
        a.part_val[blockIdx.x] = bv;
        a.part_idx[blockIdx.x] = bi;
    }
}

}  // namespace jy
