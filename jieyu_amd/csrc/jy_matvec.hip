// jy_matvec.hip — the decode-step Q8_0 matvec (one token, batch 1).
//
// Arithmetic of dot_row_avx2 (libs/matmul_libs/matmul_q.h:111-132), bit for bit:
// 32 virtual FMA lanes per row, lane L accumulates x[32b+L] * (q*d) over the
// blocks b in order, then the fixed tree
//   s[i] = (a[i]+a[8+i]) + (a[16+i]+a[24+i]),  r[i] = s[i]+s[4+i],  y = (r0+r1)+(r2+r3).
// Each thread owns two lanes of one row (16 threads per row, 4 rows per wave),
// so a row's 32 chains run in parallel and the tree is four butterflies plus an
// in-lane add.  Weights stream from HBM as 16 B per lane (1 KiB per wave per
// chunk of 8 blocks) with eight chunks in flight; the activation vector sits in
// LDS, lane-pair major.  Dequantisation is one v_fma_mix (q * fp16 scale, exact)
// per weight.  With NORM == MV_NORM_EXACT the staged vector is RMS-normalised in LDS
// first (the reference's rmsnorm), its weights prefetched while x is staged.  With
// MV_NORM_LINEAR (the tolerance mode) the staged vector is x times the norm weights, the
// sum of squares is taken in the same pass, and each finished dot is multiplied by
// 1/sqrt(ss/K + eps) (RMSNorm by linearity): no step of the weight stream waits for it.
#include <algorithm>

#include "jy_matvec.h"

namespace jy {

__device__ __forceinline__ void mv_chunk(const uint4& w, const uint4& dd, const float* xrow, int cc, float& a0,
                                         float& a1) {
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
        const float w0 = __builtin_fmaf(q0, dh, 0.0f);  // exact q*d; +0 addend only affects the sign of 0
        const float w1 = __builtin_fmaf(q1, dh, 0.0f);
        a0 = __builtin_fmaf(xv[2 * j], w0, a0);
        a1 = __builtin_fmaf(xv[2 * j + 1], w1, a1);
    }
}

// The sum of squares of one RMSNorm lane: v = fma(e, e, v) over pe[0], po[0], pe[2],
// po[2], ... (npairs of each), two LDS rows walked in step.  The LDS operands stream
// through two register sets of 4 pairs each (GCN assembly, as for the attention
// chains: in C the compiler waits on every batch's own loads); the tail is C.  The
// sets are small so the normalising matvec keeps its register budget.
__device__ __forceinline__ float norm_chain(const float* pe, const float* po, int npairs, float v) {
    int nb = npairs >> 3;
    if (nb > 0) {
        uint32_t ae = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)pe;
        uint32_t ao = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)po;
        asm volatile(
        "s_waitcnt lgkmcnt(0)\n"
        "ds_read2_b32 v[112:113], %[pe] offset0:0 offset1:2\n"
        "ds_read2_b32 v[114:115], %[pe] offset0:4 offset1:6\n"
        "ds_read2_b32 v[116:117], %[po] offset0:0 offset1:2\n"
        "ds_read2_b32 v[118:119], %[po] offset0:4 offset1:6\n"
        "ds_read2_b32 v[120:121], %[pe] offset0:8 offset1:10\n"
        "ds_read2_b32 v[122:123], %[pe] offset0:12 offset1:14\n"
        "ds_read2_b32 v[124:125], %[po] offset0:8 offset1:10\n"
        "ds_read2_b32 v[126:127], %[po] offset0:12 offset1:14\n"
        "s_sub_u32 %[nb], %[nb], 1\n"
        "L_ss_loop_%=:\n"
        "s_cmp_eq_u32 %[nb], 0\n"
        "s_cbranch_scc1 L_ss_last_%=\n"
        "s_waitcnt lgkmcnt(4)\n"
        "v_fmac_f32_e32 %[v], v112, v112\n"
        "v_fmac_f32_e32 %[v], v116, v116\n"
        "v_fmac_f32_e32 %[v], v113, v113\n"
        "v_fmac_f32_e32 %[v], v117, v117\n"
        "v_fmac_f32_e32 %[v], v114, v114\n"
        "v_fmac_f32_e32 %[v], v118, v118\n"
        "v_fmac_f32_e32 %[v], v115, v115\n"
        "v_fmac_f32_e32 %[v], v119, v119\n"
        "v_add_u32_e32 %[pe], 64, %[pe]\n"
        "v_add_u32_e32 %[po], 64, %[po]\n"
        "ds_read2_b32 v[112:113], %[pe] offset0:0 offset1:2\n"
        "ds_read2_b32 v[114:115], %[pe] offset0:4 offset1:6\n"
        "ds_read2_b32 v[116:117], %[po] offset0:0 offset1:2\n"
        "ds_read2_b32 v[118:119], %[po] offset0:4 offset1:6\n"
        "s_waitcnt lgkmcnt(4)\n"
        "v_fmac_f32_e32 %[v], v120, v120\n"
        "v_fmac_f32_e32 %[v], v124, v124\n"
        "v_fmac_f32_e32 %[v], v121, v121\n"
        "v_fmac_f32_e32 %[v], v125, v125\n"
        "v_fmac_f32_e32 %[v], v122, v122\n"
        "v_fmac_f32_e32 %[v], v126, v126\n"
        "v_fmac_f32_e32 %[v], v123, v123\n"
        "v_fmac_f32_e32 %[v], v127, v127\n"
        "ds_read2_b32 v[120:121], %[pe] offset0:8 offset1:10\n"
        "ds_read2_b32 v[122:123], %[pe] offset0:12 offset1:14\n"
        "ds_read2_b32 v[124:125], %[po] offset0:8 offset1:10\n"
        "ds_read2_b32 v[126:127], %[po] offset0:12 offset1:14\n"
        "s_sub_u32 %[nb], %[nb], 1\n"
        "s_branch L_ss_loop_%=\n"
        "L_ss_last_%=:\n"
        "s_waitcnt lgkmcnt(4)\n"
        "v_fmac_f32_e32 %[v], v112, v112\n"
        "v_fmac_f32_e32 %[v], v116, v116\n"
        "v_fmac_f32_e32 %[v], v113, v113\n"
        "v_fmac_f32_e32 %[v], v117, v117\n"
        "v_fmac_f32_e32 %[v], v114, v114\n"
        "v_fmac_f32_e32 %[v], v118, v118\n"
        "v_fmac_f32_e32 %[v], v115, v115\n"
        "v_fmac_f32_e32 %[v], v119, v119\n"
        "s_waitcnt lgkmcnt(0)\n"
        "v_fmac_f32_e32 %[v], v120, v120\n"
        "v_fmac_f32_e32 %[v], v124, v124\n"
        "v_fmac_f32_e32 %[v], v121, v121\n"
        "v_fmac_f32_e32 %[v], v125, v125\n"
        "v_fmac_f32_e32 %[v], v122, v122\n"
        "v_fmac_f32_e32 %[v], v126, v126\n"
        "v_fmac_f32_e32 %[v], v123, v123\n"
        "v_fmac_f32_e32 %[v], v127, v127\n"
        : [v] "+v"(v), [pe] "+v"(ae), [po] "+v"(ao), [nb] "+s"(nb)
        :
        : "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "scc", "memory");
    }
    for (int m = npairs & ~7; m < npairs; m++) {
        v = __builtin_fmaf(pe[2 * m], pe[2 * m], v);
        v = __builtin_fmaf(po[2 * m], po[2 * m], v);
    }
    return v;
}

// one wave owns row groups wid, wid + TW, ... (TW = waves in the grid), `per` of
// them; the chunk stream of consecutive row groups is pipelined without a gap.
template <int EPI, int NORM, int MV_U>
__global__ __launch_bounds__(256) void matvec_q8_kernel(Q8Dev W, const float* __restrict__ x,
                                                        const float* __restrict__ nw, float* __restrict__ out,
                                                        MvArgs a, int per) {
    // [16][XS]: lane pair g, block b, lane c.  16-byte alignment keeps the ds_read_b128
    // of the main loop aligned whatever static LDS the epilogue adds.
    extern __shared__ __align__(16) float xs[];
    __shared__ float red[18];
    __shared__ float ssw[4];
    constexpr bool EXN = NORM == MV_NORM_EXACT, LIN = NORM == MV_NORM_LINEAR;
    __shared__ float rowv[64];
    __shared__ int rowi[64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwv = blockDim.x >> 6;
    // the wave index is uniform: computed from readfirstlane, every chunk address is
    // scalar (a scalar base plus the lane's fixed offset)
    const int wid = blockIdx.x * nwv + __builtin_amdgcn_readfirstlane(wave);
    const int r = lane >> 4, g = lane & 15;
    const int K = W.cols, nch = W.nch, nchp = W.nchp, XS = 2 * W.nbp + 4;
    const int groups = (W.rows + 3) >> 2;

    // this wave's row groups are wid, wid+TW, ... (TW = waves in the grid), so the waves
    // in flight read neighbouring row groups.  The wave's weight stream runs through
    // each row group's nchp stored chunks (those past nch are zero and never computed)
    // and jumps to its next row group; nchp is a multiple of the batch size, so a batch
    // never straddles two.  Chunk offsets are scalar (buffer loads with the lane's fixed
    // offset in a register), clamped so loads past the matrix stay in its zero tail.
    const int TW = gridDim.x * nwv;
    const int cmax = groups * nchp + 8 - MV_U;
    int lrg = wid, lp = 0;  // row group and chunk of the next load
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(W.qs, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(W.d, (short)0, 0x7fffffff, 0x00020000);
    const int qoff = lane * 16, doff = r * 16;
    auto load = [&](uint4* wb, uint4* db) {
        const int c = min(lrg * nchp + lp, cmax);
#pragma unroll
        for (int u = 0; u < MV_U; u++) {
            wb[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qrs, qoff, (c + u) * 1024, 0));
            db[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(drs, doff, (c + u) * 64, 0));
        }
        lp += MV_U;
        if (lp == nchp) {
            lp = 0;
            lrg = min(lrg + TW, groups);
        }
    };

    // stage x (and with NORM the RMSNorm weights, into nws behind the staged vector),
    // four floats per load, several loads in flight per thread; zero past K, so
    // padding blocks contribute exact zeros.  The vector's first batch is requested
    // before the weight prefetch so it does not queue behind it.  Without NORM both
    // weight buffers follow it at once; with NORM only the first does, and the second
    // once the vector is in (a full prefetch ahead of the vector's later loads delays
    // them).  The buffers then stay two ahead of the compute.
    uint4 wA[MV_U], dA[MV_U], wB[MV_U], dB[MV_U];
    float* nws = xs + 16 * XS;
    const int nk4 = K / 4;
    {
        const int nv4 = W.nbp * 8;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const float4* w4 = reinterpret_cast<const float4*>(nw);
        constexpr int SU = NORM ? 4 : 8;  // loads per thread per batch (x and w with NORM)
        float ss = 0.0f;
        for (int b0 = 0; b0 < nv4; b0 += SU * blockDim.x) {
            float4 v[SU], wv[SU];
#pragma unroll
            for (int u = 0; u < SU; u++) {
                const int i = b0 + tid + u * blockDim.x;
                v[u] = (i < nv4 && i < nk4) ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (NORM) wv[u] = i < nk4 ? w4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            if (b0 == 0) {
                load(wA, dA);
                if (!EXN) load(wB, dB);
            }
#pragma unroll
            for (int u = 0; u < SU; u++) {
                const int i = b0 + tid + u * blockDim.x;
                if (i < nv4) {
                    const int k = 4 * i;
                    float4 e = v[u];
                    if (LIN) {
                        ss = __builtin_fmaf(e.x, e.x, ss);
                        ss = __builtin_fmaf(e.y, e.y, ss);
                        ss = __builtin_fmaf(e.z, e.z, ss);
                        ss = __builtin_fmaf(e.w, e.w, ss);
                        e = make_float4(e.x * wv[u].x, e.y * wv[u].y, e.z * wv[u].z, e.w * wv[u].w);
                    }
                    xs[xs_index(k, XS)] = e.x;
                    xs[xs_index(k + 1, XS)] = e.y;
                    xs[xs_index(k + 2, XS)] = e.z;
                    xs[xs_index(k + 3, XS)] = e.w;
                    if (EXN && i < nk4) reinterpret_cast<float4*>(nws)[i] = wv[u];
                }
            }
        }
        if (LIN) {
            ss += __shfl_xor(ss, 1);
            ss += __shfl_xor(ss, 2);
            ss += __shfl_xor(ss, 4);
            ss += __shfl_xor(ss, 8);
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if (lane == 0) ssw[wave] = ss;
        }
    }
    lds_barrier();  // the weight prefetch stays in flight
    float nscale = 1.0f;
    bool nzero = false;
    if (LIN) {
        const float tot = (ssw[0] + ssw[1]) + (ssw[2] + ssw[3]);
        const float den = tot / (float)K + 1e-5f;
        nzero = !(den > 0.0f);
        nscale = nzero ? 0.0f : 1.0f / sqrtf(den);
    }
    if (EXN) {
        // the second weight buffer, now that the vector is in: the weights are first
        // needed after the normalisation
        load(wB, dB);
        // RMSNorm of the staged vector (libs/model_libs/rmsnorm/x86/x86_classic.txt:2-26):
        // lanes 0..15 of wave 0 run the 16 FMA chains (lane l: elements 16c+l, an 8-wide
        // remainder pass feeds lanes 0..7), the fold ((v0+v1) -> halves -> two hadds) is
        // four butterflies, lane 0 adds the tail, then x = (x*scale)*w with the staged weights
        if (wave == 0) {
            const int n16 = K / 16 * 16;
            const bool rem8 = n16 + 8 <= K;
            // element 16c + l sits at xs_index = (8(c&1) + l/2)*XS + 2(c/2) + (l&1): two
            // running addresses per lane, one for even c and one for odd c
            float v = 0.0f;
            if (lane < 16) {
                const float* pe = xs + (lane >> 1) * XS + (lane & 1);
                const float* po = pe + 8 * XS;
                const int npairs = n16 >> 5;
                v = norm_chain(pe, po, npairs, v);
                if (n16 & 16) {  // an odd number of 16-element groups ends on an even c
                    const float e = pe[2 * npairs];
                    v = __builtin_fmaf(e, e, v);
                }
                if (lane < 8 && rem8) {
                    const float e = xs[xs_index(n16 + lane, XS)];
                    v = __builtin_fmaf(e, e, v);
                }
            }
            // fold ((v0+v1) -> halves -> two hadds) as butterflies; every add of the tree
            // is commutative, so lane 0 ends with the reference's value bit for bit
            float t = v + dpp_f<0x128>(v);    // s[i] = v[i] + v[8+i]
            t = t + dpp_f<0x12C>(t);          // q[i] = s[i] + s[4+i]
            t = t + dpp_f<0xB1>(t);           // q0+q1 (lane 0), q2+q3 (lane 2)
            float ss = t + dpp_f<0x4E>(t);    // (q0+q1) + (q2+q3)
            if (lane == 0) {
                // the scalar tail as GCC builds it: with four or more left, the first four
                // squares are rounded products added in order, the rest fused
                int k = n16 + (rem8 ? 8 : 0);
                if (K - k >= 4)
                    for (const int e = k + 4; k < e; k++) {
                        const float q = xs[xs_index(k, XS)];
                        ss = ss + q * q;
                    }
                for (; k < K; k++) {
                    const float q = xs[xs_index(k, XS)];
                    ss = __builtin_fmaf(q, q, ss);
                }
                const float den = ss / (float)K + 1e-5f;
                red[17] = den <= 0.0f ? 1.0f : 0.0f;
                red[16] = den <= 0.0f ? 0.0f : 1.0f / sqrtf(den);
            }
        }
        lds_barrier();
        const float scale = red[16];
        const bool zero = red[17] != 0.0f;
        // x = (x*scale)*w: a thread's four-element groups, all reads before the writes
        for (int b0 = 0; b0 < nk4; b0 += 4 * blockDim.x) {
            float xv[4][4];
            float4 wv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = b0 + tid + u * blockDim.x;
                if (i < nk4) {
                    wv[u] = reinterpret_cast<const float4*>(nws)[i];
#pragma unroll
                    for (int c = 0; c < 4; c++) xv[u][c] = xs[xs_index(4 * i + c, XS)];
                }
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = b0 + tid + u * blockDim.x;
                if (i < nk4) {
                    const float w4[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        xs[xs_index(4 * i + c, XS)] = zero ? 0.0f : (xv[u][c] * scale) * w4[c];
                }
            }
        }
        lds_barrier();
    }

    const float* xrow = xs + g * XS;
    float best_v = -__builtin_inff();
    int best_i = 0x7fffffff;
    for (int it = 0; it < per; it++) {
        const int rg = wid + it * TW;
        const bool active = rg < groups;
        const int row = rg * 4 + r;
        const bool own = active && g == 0 && row < W.rows;
        const MvPre pre = mv_preload<EPI>(row, own, r, a, out);
        float a0 = 0.0f, a1 = 0.0f;
        for (int ch = 0; ch < nchp; ch += 2 * MV_U) {
            if (active) {
#pragma unroll
                for (int u = 0; u < MV_U; u++)
                    if (ch + u < nch) mv_chunk(wA[u], dA[u], xrow, ch + u, a0, a1);
            }
            load(wA, dA);
            if (active) {
#pragma unroll
                for (int u = 0; u < MV_U; u++)
                    if (ch + MV_U + u < nch) mv_chunk(wB[u], dB[u], xrow, ch + MV_U + u, a0, a1);
            }
            load(wB, dB);
        }
        // lanes 2g, 2g+1 -> the reference's reduction tree
        // (row rotations give lane g the lanes g+4 and g+8 of its 16-lane row: the
        // partners g ^ 4, g ^ 8 of the lanes the tree keeps)
        a0 += dpp_f<0x12C>(a0);
        a1 += dpp_f<0x12C>(a1);
        a0 += dpp_f<0x128>(a0);
        a1 += dpp_f<0x128>(a1);
        a0 += dpp_f<0x4E>(a0);
        a1 += dpp_f<0x4E>(a1);
        const float t = a0 + a1;
        float y = t + dpp_f<0xB1>(t);
        if (LIN) y = nzero ? 0.0f : y * nscale;
        mv_epilogue<EPI>(y, row, own, r, W.rows, a, out, best_v, best_i, &pre);
    }

    if (EPI == EPI_ARGMAX) mv_argmax_partial(best_v, best_i, g, r, wave, nwv, rowv, rowi, a);
}

// the greedy pick over the lm_head workgroups' partial maxima: lowest index among
// equal values (the reference's first strict maximum), then ids[len] = pick, len++,
// and the stop flag on an EOS id (generate.h:57-60, :78-83)
__global__ __launch_bounds__(256) void argmax_finish_kernel(const float* __restrict__ part_val,
                                                            const int* __restrict__ part_idx, int np, int* ids,
                                                            int* mstate, const int* eos, int neos) {
    __shared__ float wv[4];
    __shared__ int wi[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    for (int i = tid; i < np; i += blockDim.x) {
        const float v = part_val[i];
        const int ix = part_idx[i];
        if (v > bv || (v == bv && ix < bi)) {
            bv = v;
            bi = ix;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        wv[wave] = bv;
        wi[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        bv = wv[0];
        bi = wi[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++)
            if (wv[w] > bv || (wv[w] == bv && wi[w] < bi)) {
                bv = wv[w];
                bi = wi[w];
            }
        if (bi == 0x7fffffff) bi = 0;
        if (!mstate[1]) {
            const int len = mstate[0];
            ids[len] = bi;
            mstate[0] = len + 1;
            for (int e = 0; e < neos; e++)
                if (bi == eos[e]) mstate[1] = 1;
        }
    }
}

void launch_argmax_finish(const MvArgs& a, int np, hipStream_t st) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(256), 0, st, a.part_val, a.part_idx, np, a.ids, a.mstate,
                       a.eos, a.neos);
}

static int g_cus = 256;

// launch shape: 4 waves per workgroup, at most 4 workgroups per CU; each wave owns
// `per` row groups so the prologue (staging, RMSNorm) is paid once per workgroup.  With
// two row groups per wave the grid is every slot (4 workgroups per CU) and the row groups
// are strided over all its waves, so every CU gets the same share: sized to the row groups
// instead, 28672 x 4096 took 896 workgroups, 4 on half the CUs and 3 on the others, and ran
// 27.7 us against 26.2 (Llama-3-8B decode 436.5 -> 446.3 tokens/s).  With three or more
// (Qwen2.5-7B's 37888-row gate/up, the lm_heads) the full grid measured slightly slower
// (Qwen2.5-7B decode 412.9 vs 409.5, Qwen2.5-0.5B 1416.5 vs 1410.8): its extra workgroups
// stage the vector again for less work each.
static void mv_shape(const Q8Dev& W, bool exn, int* grid, int* per) {
    const int nwv = 4;
    const int groups = (W.rows + 3) / 4;
    const int max_waves = 4 * g_cus * nwv;
    *per = (groups + max_waves - 1) / max_waves;
    *grid = (groups + nwv * *per - 1) / (nwv * *per);
    const size_t lds = ((size_t)16 * (2 * W.nbp + 4) + (exn ? (size_t)W.cols : 0)) * sizeof(float);
    if (*per == 2 && 4 * lds <= matvec_lds_limit()) *grid = max_waves / nwv;
}

// workgroups of an lm_head launch (one partial maximum each), normalising or not
int argmax_partials(int rows) {
    Q8Dev w;
    w.rows = rows;
    int grid = 0, per = 0, g2 = 0;
    mv_shape(w, false, &grid, &per);
    mv_shape(w, true, &g2, &per);
    return std::max(grid, g2);
}

template <int EPI, int NORM>
static void mv_launch(const Q8Dev& W, const float* x, const float* nw, float* out, const MvArgs& a, hipStream_t st) {
    int grid, per;
    mv_shape(W, NORM == MV_NORM_EXACT, &grid, &per);
    const size_t lds = ((size_t)16 * (2 * W.nbp + 4) + (NORM == MV_NORM_EXACT ? (size_t)W.cols : 0)) * sizeof(float);
    if (W.U == 4)
        hipLaunchKernelGGL((matvec_q8_kernel<EPI, NORM, 4>), dim3(grid), dim3(256), lds, st, W, x, nw, out, a, per);
    else if (W.U == 2)
        hipLaunchKernelGGL((matvec_q8_kernel<EPI, NORM, 2>), dim3(grid), dim3(256), lds, st, W, x, nw, out, a, per);
    else
        hipLaunchKernelGGL((matvec_q8_kernel<EPI, NORM, 1>), dim3(grid), dim3(256), lds, st, W, x, nw, out, a, per);
    if (EPI == EPI_ARGMAX) launch_argmax_finish(a, grid, st);
}

template <int NORM>
static void mv_dispatch(const Q8Dev& W, const float* x, const float* nw, float* out, Epi epi, const MvArgs& a,
                        hipStream_t st) {
    switch (epi) {
    case EPI_STORE: mv_launch<EPI_STORE, NORM>(W, x, nw, out, a, st); break;
    case EPI_BIAS: mv_launch<EPI_BIAS, NORM>(W, x, nw, out, a, st); break;
    case EPI_RESID: mv_launch<EPI_RESID, NORM>(W, x, nw, out, a, st); break;
    case EPI_SWIGLU: mv_launch<EPI_SWIGLU, NORM>(W, x, nw, out, a, st); break;
    case EPI_ROPE: mv_launch<EPI_ROPE, NORM>(W, x, nw, out, a, st); break;
    case EPI_ARGMAX: mv_launch<EPI_ARGMAX, NORM>(W, x, nw, out, a, st); break;
    }
}

void launch_matvec_q8(const Q8Dev& W, const float* x, const float* norm_w, float* out, Epi epi, const MvArgs& a,
                      hipStream_t st, bool norm_linear) {
    if (norm_w && norm_linear)
        mv_dispatch<MV_NORM_LINEAR>(W, x, norm_w, out, epi, a, st);
    else if (norm_w)
        mv_dispatch<MV_NORM_EXACT>(W, x, norm_w, out, epi, a, st);
    else
        mv_dispatch<MV_NORM_NONE>(W, x, nullptr, out, epi, a, st);
}

size_t matvec_lds_bytes(int cols, bool norm) {
    const Q8Dev w = q8_shape(1, cols);
    return ((size_t)16 * (2 * w.nbp + 4) + (norm ? (size_t)cols : 0)) * sizeof(float);
}
size_t matvec_lds_limit() { return 160 * 1024 - 2048; }

template <int EPI, int NORM>
static hipError_t mv_attr() {
    hipError_t e = hipSuccess;
    for (const void* f : {reinterpret_cast<const void*>(&matvec_q8_kernel<EPI, NORM, 4>),
                          reinterpret_cast<const void*>(&matvec_q8_kernel<EPI, NORM, 2>),
                          reinterpret_cast<const void*>(&matvec_q8_kernel<EPI, NORM, 1>)})
        if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 2048);
    return e;
}

hipError_t matvec_init() {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    if (cus > 0) g_cus = cus;
    for (hipError_t r : {mv_attr<EPI_STORE, 0>(), mv_attr<EPI_BIAS, 0>(), mv_attr<EPI_RESID, 0>(),
                         mv_attr<EPI_SWIGLU, 0>(), mv_attr<EPI_ROPE, 0>(), mv_attr<EPI_ARGMAX, 0>(),
                         mv_attr<EPI_STORE, 1>(), mv_attr<EPI_BIAS, 1>(), mv_attr<EPI_RESID, 1>(),
                         mv_attr<EPI_SWIGLU, 1>(), mv_attr<EPI_ROPE, 1>(), mv_attr<EPI_ARGMAX, 1>(),
                         mv_attr<EPI_STORE, 2>(), mv_attr<EPI_BIAS, 2>(), mv_attr<EPI_RESID, 2>(),
                         mv_attr<EPI_SWIGLU, 2>(), mv_attr<EPI_ROPE, 2>(), mv_attr<EPI_ARGMAX, 2>()})
        if (r != hipSuccess && e == hipSuccess) e = r;
    return e;
}

}  // namespace jy
