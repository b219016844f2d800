// jy_matvec_split.hip — the decode Q8_0 matvec in the tolerance mode: each row's dot
// y[n] = sum_k x[k] * q[n][k] * d[n][k/32] (libs/matmul_libs/matmul_q.h:101-144) split
// over SK waves of a workgroup, each taking a slice of the row's blocks, with a free
// summation order inside a slice.  Dequantisation stays exact (int8 times the fp16
// block scale); only the fp32 rounding of the sums differs from dot_row_avx2.
//
// Weights are the lane-pair layout of jy_layout.h (row groups of 4 rows x chunks of 8
// blocks, 1 KiB + 64 B per chunk), read as 16 B per lane with a ring of two U-chunk
// register buffers.  A wave's stream is its row groups' slices back to back; a row
// group's SK slices are reduced through LDS by the wave with slice 0, which runs the
// epilogue.
//
// With NORM the kernel applies RMSNorm (libs/model_libs/rmsnorm/rmsnorm.h:8-78,
// eps 1e-5) by linearity: it stages x * w (the norm weights) and the sum of x^2 in the
// same pass, and multiplies each finished dot by 1/sqrt(ss/K + eps).  No step of the
// weight stream waits for the normalisation.
#include <algorithm>

#include "jy_matvec.h"

namespace jy {

// one chunk of one lane: blocks j = 0..7, lanes 2g, 2g+1 of each: acc += d_j * (x0 q0 + x1 q1)
__device__ __forceinline__ float split_chunk_dot(const uint4& w, const uint4& dd, const float* xrow, int cc,
                                                 float acc) {
    const float4* xp = reinterpret_cast<const float4*>(xrow + cc * 16);
    const float4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
    const float xv[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                          x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    const uint32_t dv[4] = {dd.x, dd.y, dd.z, dd.w};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t word = wv[j >> 1];
        const int sh = (j & 1) * 16;
        const float q0 = (float)(int8_t)(word >> sh);
        const float q1 = (float)(int8_t)(word >> (sh + 8));
        const float dh = (float)__builtin_bit_cast(_Float16, (uint16_t)(dv[j >> 1] >> sh));
        const float t = __builtin_fmaf(xv[2 * j + 1], q1, xv[2 * j] * q0);
        acc = __builtin_fmaf(t, dh, acc);
    }
    return acc;
}

// Wave w of a workgroup: slice ks = w % SK of row group rs = w / SK of each of the
// workgroup's passes; pass p covers row groups (p * gridDim.x + blockIdx.x) * RPW + rs.
// cps = nchp / SK chunks per slice, streamed in steps of U chunks; the last step of a
// slice may be partial (its spare loads land on in-bounds chunks that are not used).
template <int EPI, bool NORM, int SK, int U>
__global__ __launch_bounds__(256) void matvec_q8_split_kernel(Q8Dev W, const float* __restrict__ x,
                                                              const float* __restrict__ nw, float* __restrict__ out,
                                                              MvArgs a, int per) {
    constexpr int NWV = 4, RPW = NWV / SK;
    extern __shared__ __align__(16) float xs[];
    __shared__ float red[2][NWV][4];
    __shared__ float ssw[NWV];
    __shared__ float rowv[64];
    __shared__ int rowi[64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int ks = wv % SK, rs = wv / SK;
    const int r = lane >> 4, g = lane & 15;
    const int K = W.cols, nch = W.nch, nchp = W.nchp, XS = 2 * W.nbp + 4;
    const int groups = (W.rows + 3) >> 2;
    const int cps = nchp / SK, c_lo = ks * cps;
    const int steps_per_row = (cps + U - 1) / U;

    // the weight stream: (row group of pass p, chunk c_lo + i), i < cps, pass after pass
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(W.qs, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(W.d, (short)0, 0x7fffffff, 0x00020000);
    const int qoff = lane * 16, doff = r * 16;
    const int cmax = groups * nchp + 8 - U;  // loads past the matrix stay in its zero tail
    int lp = 0, li = 0;                      // pass and chunk offset of the next load
    auto rg_of = [&](int p) { return (p * (int)gridDim.x + (int)blockIdx.x) * RPW + rs; };
    auto load = [&](uint4* wb, uint4* db) {
        const int c = min(min(rg_of(lp), groups) * nchp + c_lo + li, cmax);
#pragma unroll
        for (int u = 0; u < U; u++) {
            wb[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qrs, qoff, (c + u) * 1024, 0));
            db[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(drs, doff, (c + u) * 64, 0));
        }
        li += U;
        if (li >= cps) {
            li = 0;
            lp++;
        }
    };
    uint4 wA[U], dA[U], wB[U], dB[U];
    load(wA, dA);
    load(wB, dB);

    // stage x (times the norm weights with NORM) while the first buffers are in flight;
    // zero past K so padding blocks add exact zeros; with NORM each thread also sums
    // the squares of the elements it stages
    float ss = 0.0f;
    {
        const int nv4 = W.nbp * 8, nk4 = K / 4;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const float4* w4 = reinterpret_cast<const float4*>(nw);
        for (int b0 = 0; b0 < nv4; b0 += 4 * 256) {
            float4 v[4], wt[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = b0 + tid + u * 256;
                const bool in = i < nv4 && i < nk4;
                v[u] = in ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (NORM) wt[u] = in ? w4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = b0 + tid + u * 256;
                if (i < nv4) {
                    const int k = 4 * i;
                    float4 e = v[u];
                    if (NORM) {
                        ss = __builtin_fmaf(e.x, e.x, ss);
                        ss = __builtin_fmaf(e.y, e.y, ss);
                        ss = __builtin_fmaf(e.z, e.z, ss);
                        ss = __builtin_fmaf(e.w, e.w, ss);
                        e = make_float4(e.x * wt[u].x, e.y * wt[u].y, e.z * wt[u].z, e.w * wt[u].w);
                    }
                    xs[xs_index(k, XS)] = e.x;
                    xs[xs_index(k + 1, XS)] = e.y;
                    xs[xs_index(k + 2, XS)] = e.z;
                    xs[xs_index(k + 3, XS)] = e.w;
                }
            }
        }
    }
    if (NORM) {
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        ss += __shfl_xor(ss, 8);
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (lane == 0) ssw[wave] = ss;
    }
    lds_barrier();  // the weight loads stay in flight
    float nscale = 1.0f;
    bool nzero = false;
    if (NORM) {
        const float tot = (ssw[0] + ssw[1]) + (ssw[2] + ssw[3]);
        const float den = tot / (float)K + 1e-5f;
        nzero = !(den > 0.0f);
        nscale = nzero ? 0.0f : 1.0f / sqrtf(den);
    }

    const float* xrow = xs + g * XS;
    float best_v = -__builtin_inff();
    int best_i = 0x7fffffff;
    float acc = 0.0f;
    int par = 0;
    // the epilogue's per-row operands of a pass, requested when its stream starts
    auto preload = [&](int p) {
        const int rg = rg_of(p), row = rg * 4 + r;
        return ks == 0 ? mv_preload<EPI>(row, rg < groups && g == 0 && row < W.rows, r, a, out) : MvPre();
    };
    MvPre pre = preload(0);
    // one finished row-group slice: fold the 16 lanes of each row, then the SK slices
    auto finish = [&](int p) {
        acc += dpp_f<0x128>(acc);  // l + 8
        acc += dpp_f<0x124>(acc);  // l + 12 (l - 4)
        acc += dpp_f<0x4E>(acc);   // l ^ 2
        acc += dpp_f<0xB1>(acc);   // l ^ 1: every lane of the row holds the row's sum
        float y = acc;
        if (SK > 1) {
            if (g == 0) red[par][wv][r] = acc;
            lds_barrier();
            if (ks == 0) {
                y = red[par][rs * SK][r];
#pragma unroll
                for (int k = 1; k < SK; k++) y += red[par][rs * SK + k][r];
            }
            par ^= 1;
        }
        if (ks == 0) {
            const int rg = rg_of(p);
            const int row = rg * 4 + r;
            const bool own = rg < groups && g == 0 && row < W.rows;
            if (NORM) y = nzero ? 0.0f : y * nscale;
            mv_epilogue<EPI>(y, row, own, r, W.rows, a, out, best_v, best_i, &pre);
        }
        if (p + 1 < per) pre = preload(p + 1);
        acc = 0.0f;
    };

    // the stream: buffers A and B alternate; a row-group slice ends every steps_per_row
    const int nsteps = per * steps_per_row;
    int ci = 0;  // chunk index within the current slice
    for (int s = 0; s < nsteps; s += 2) {
        {
            const int p = s / steps_per_row;
#pragma unroll
            for (int u = 0; u < U; u++)
                if (ci + u < cps && c_lo + ci + u < nch) acc = split_chunk_dot(wA[u], dA[u], xrow, c_lo + ci + u, acc);
            load(wA, dA);
            ci += U;
            if (ci >= cps) {
                finish(p);
                ci = 0;
            }
        }
        if (s + 1 < nsteps) {
            const int p = (s + 1) / steps_per_row;
#pragma unroll
            for (int u = 0; u < U; u++)
                if (ci + u < cps && c_lo + ci + u < nch) acc = split_chunk_dot(wB[u], dB[u], xrow, c_lo + ci + u, acc);
            load(wB, dB);
            ci += U;
            if (ci >= cps) {
                finish(p);
                ci = 0;
            }
        }
    }

    if (EPI == EPI_ARGMAX) mv_argmax_partial(best_v, best_i, g, r, wave, NWV, rowv, rowi, a);
}

static int g_split_cus = 256;

struct SplitShape {
    int SK, U, grid, per;
};

// the deepest buffer of U in {8, 7, 4, 2, 1} chunks that divides a slice of cps chunks
static int split_u(int cps) {
    for (int u : {8, 7, 4, 2})
        if (cps % u == 0) return u;
    return 1;
}

static SplitShape shape_of(const Q8Dev& W, int sk, int wpc) {
    const int groups = (W.rows + 3) / 4;
    SplitShape s{sk, split_u(W.nchp / sk), 1, 1};
    const int rpw = 4 / sk;
    const int passes = (groups + rpw - 1) / rpw;
    const int max_wg = wpc * g_split_cus;
    s.per = (passes + max_wg - 1) / max_wg;
    s.grid = (passes + s.per - 1) / s.per;
    return s;
}

// split and buffer depth by shape: enough waves to keep the matrix's bytes in flight
// (at least two per SIMD), each slice a whole number of buffers
static SplitShape split_shape(const Q8Dev& W) {
    const int groups = (W.rows + 3) / 4;
    int sk = 1;
    while (sk < 4 && groups * sk < 8 * g_split_cus && W.nchp % (sk * 2) == 0) sk *= 2;
    return shape_of(W, sk, 4);
}

template <int EPI, bool NORM, int SK>
static void split_launch_u(const Q8Dev& W, const SplitShape& sh, const float* x, const float* nw, float* out,
                           const MvArgs& a, size_t lds, hipStream_t st) {
    if (sh.U == 8)
        hipLaunchKernelGGL((matvec_q8_split_kernel<EPI, NORM, SK, 8>), dim3(sh.grid), dim3(256), lds, st, W, x, nw,
                           out, a, sh.per);
    else if (sh.U == 7)
        hipLaunchKernelGGL((matvec_q8_split_kernel<EPI, NORM, SK, 7>), dim3(sh.grid), dim3(256), lds, st, W, x, nw,
                           out, a, sh.per);
    else if (sh.U == 4)
        hipLaunchKernelGGL((matvec_q8_split_kernel<EPI, NORM, SK, 4>), dim3(sh.grid), dim3(256), lds, st, W, x, nw,
                           out, a, sh.per);
    else if (sh.U == 2)
        hipLaunchKernelGGL((matvec_q8_split_kernel<EPI, NORM, SK, 2>), dim3(sh.grid), dim3(256), lds, st, W, x, nw,
                           out, a, sh.per);
    else
        hipLaunchKernelGGL((matvec_q8_split_kernel<EPI, NORM, SK, 1>), dim3(sh.grid), dim3(256), lds, st, W, x, nw,
                           out, a, sh.per);
}

void launch_argmax_finish(const MvArgs& a, int np, hipStream_t st);

template <int EPI, bool NORM>
static void split_launch(const Q8Dev& W, const float* x, const float* nw, float* out, const MvArgs& a,
                         hipStream_t st) {
    const SplitShape sh = split_shape(W);
    const size_t lds = (size_t)16 * (2 * W.nbp + 4) * sizeof(float);
    if (sh.SK == 4)
        split_launch_u<EPI, NORM, 4>(W, sh, x, nw, out, a, lds, st);
    else if (sh.SK == 2)
        split_launch_u<EPI, NORM, 2>(W, sh, x, nw, out, a, lds, st);
    else
        split_launch_u<EPI, NORM, 1>(W, sh, x, nw, out, a, lds, st);
    if (EPI == EPI_ARGMAX) launch_argmax_finish(a, sh.grid, st);
}

template <bool NORM>
static void split_dispatch(const Q8Dev& W, const float* x, const float* nw, float* out, Epi epi, const MvArgs& a,
                           hipStream_t st) {
    switch (epi) {
    case EPI_STORE: split_launch<EPI_STORE, NORM>(W, x, nw, out, a, st); break;
    case EPI_BIAS: split_launch<EPI_BIAS, NORM>(W, x, nw, out, a, st); break;
    case EPI_RESID: split_launch<EPI_RESID, NORM>(W, x, nw, out, a, st); break;
    case EPI_SWIGLU: split_launch<EPI_SWIGLU, NORM>(W, x, nw, out, a, st); break;
    case EPI_ROPE: split_launch<EPI_ROPE, NORM>(W, x, nw, out, a, st); break;
    case EPI_ARGMAX: split_launch<EPI_ARGMAX, NORM>(W, x, nw, out, a, st); break;
    }
}

void launch_matvec_q8_split(const Q8Dev& W, const float* x, const float* norm_w, float* out, Epi epi,
                            const MvArgs& a, hipStream_t st) {
    if (norm_w)
        split_dispatch<true>(W, x, norm_w, out, epi, a, st);
    else
        split_dispatch<false>(W, x, nullptr, out, epi, a, st);
}

int split_argmax_partials(int rows) {
    Q8Dev w = q8_shape(rows, 32);
    return split_shape(w).grid;
}

template <int EPI, bool NORM, int SK>
static hipError_t split_attr_sk() {
    hipError_t e = hipSuccess;
    for (const void* f : {reinterpret_cast<const void*>(&matvec_q8_split_kernel<EPI, NORM, SK, 8>),
                          reinterpret_cast<const void*>(&matvec_q8_split_kernel<EPI, NORM, SK, 7>),
                          reinterpret_cast<const void*>(&matvec_q8_split_kernel<EPI, NORM, SK, 4>),
                          reinterpret_cast<const void*>(&matvec_q8_split_kernel<EPI, NORM, SK, 2>),
                          reinterpret_cast<const void*>(&matvec_q8_split_kernel<EPI, NORM, SK, 1>)})
        if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 4096);
    return e;
}

template <int EPI, bool NORM>
static hipError_t split_attr() {
    hipError_t e = split_attr_sk<EPI, NORM, 1>();
    if (e == hipSuccess) e = split_attr_sk<EPI, NORM, 2>();
    if (e == hipSuccess) e = split_attr_sk<EPI, NORM, 4>();
    return e;
}

hipError_t matvec_split_init() {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    if (cus > 0) g_split_cus = cus;
    for (hipError_t r : {split_attr<EPI_STORE, false>(), split_attr<EPI_BIAS, false>(), split_attr<EPI_RESID, false>(),
                         split_attr<EPI_SWIGLU, false>(), split_attr<EPI_ROPE, false>(), split_attr<EPI_ARGMAX, false>(),
                         split_attr<EPI_STORE, true>(), split_attr<EPI_BIAS, true>(), split_attr<EPI_RESID, true>(),
                         split_attr<EPI_SWIGLU, true>(), split_attr<EPI_ROPE, true>(), split_attr<EPI_ARGMAX, true>()})
        if (r != hipSuccess && e == hipSuccess) e = r;
    return e;
}

}  // namespace jy
