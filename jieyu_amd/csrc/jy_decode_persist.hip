// jy_decode_persist.hip — one decode token's whole layer stack (and the final norm,
// lm_head and greedy pick) as one persistent kernel, in the tolerance mode (split-dot
// matvecs, split attention).  It computes what transformer_layer x L + the head do
// (libs/model_libs/transformer_layer.h:10-90, forward.h:67-94, generate.h:48-60) with
// the arithmetic of jy_matvec_split.hip and jy_attention_split.h.
//
// Why one kernel: every kernel boundary in the decode graph costs a few microseconds of
// launch, ramp-up and drain in which HBM idles, about 200 times a token.  Here one
// workgroup per CU streams the weights of all matrices in order, and the phases of a
// layer hand their activations to each other through the agent-coherent level (sc1 loads
// and stores), separated by grid barriers: each workgroup stores its flag once its
// stores are complete, then issues the next matrix's first loads, then waits for every
// flag.  The weight stream therefore keeps running while a barrier resolves.
//
// Phases of a layer: QKV (RMSNorm by linearity, bias, RoPE) -> attention slices, the
// last slice of each kv head merging the group's slices -> O + residual -> gate/up
// (RMSNorm, SwiGLU) -> down + residual.  Then final RMSNorm + lm_head with per-workgroup
// maxima, and workgroup 0 picks the token.
//
// All workgroups must be resident at once (the launch uses one per CU, checked against
// the occupancy the runtime reports).  Every wait is bounded: a barrier that has not
// resolved after PK_SPIN polls sets the error word and stops waiting, so the grid always
// drains; the host then reports the step as failed.
#include <algorithm>

#include "jy_attention_split.h"
#include "jy_matvec.h"

namespace jy {

static constexpr int PK_THREADS = 256;
static constexpr int PK_UMAX = 8;
static constexpr int PK_SPIN = 1 << 18;

// ---------------------------------------------------------------- grid barrier

struct PkSync {
    unsigned* flags;  // [gridDim.x], zero at launch
    int* err;
};

// this workgroup's stores are complete: publish epoch
__device__ __forceinline__ void pk_arrive(const PkSync& s, unsigned epoch) {
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt 0: this wave's stores have reached the coherent level
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(s.flags + blockIdx.x, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// wait until every workgroup has published epoch (wave 0 polls; bounded)
__device__ __forceinline__ void pk_wait(const PkSync& s, unsigned epoch, int* dead) {
    if (threadIdx.x < 64 && !*dead) {
        const int nwg = gridDim.x;
        int n = 0;
        for (;;) {
            unsigned lo = 0xffffffffu;
            for (int i = threadIdx.x; i < nwg; i += 64) {
                const unsigned f = __hip_atomic_load(s.flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                lo = f < lo ? f : lo;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const unsigned t = __shfl_xor(lo, o);
                lo = t < lo ? t : lo;
            }
            if (lo >= epoch) break;
            if (++n > PK_SPIN) {
                if (threadIdx.x == 0) {
                    __hip_atomic_store(s.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    *dead = 1;
                }
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    lds_barrier();
}

// ---------------------------------------------------------------- activation staging

// x (n floats, written by other workgroups) into LDS in the lane-pair layout (zero past n
// up to nbp blocks), times the norm weights w with NORM; returns 1/sqrt(sum x^2 / n + eps)
// with NORM (1 otherwise) and sets *zero where the reference's den <= 0 zeroes the output.
template <bool NORM>
__device__ __forceinline__ float pk_stage(const float* x, int n, int nbp, const float* __restrict__ w, float* xs,
                                          float* ssw, bool* zero) {
    constexpr int PB = 8;  // float4 loads per thread in flight
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int XS = 2 * nbp + 4, nv4 = nbp * 8, n4 = n / 4;  // n is a multiple of 4 (hidden, q_dim, ffn)
    // sc1: the loads read through to the agent-coherent level, where the other workgroups'
    // sc1 stores landed (the L2 of this XCD may hold a stale line)
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, 0x7fffffff, 0x00020000);
    float ss = 0.0f;
    for (int b0 = 0; b0 < nv4; b0 += PB * PK_THREADS) {
        float4 v[PB], wt[PB];
#pragma unroll
        for (int u = 0; u < PB; u++) {
            const int i = b0 + tid + u * PK_THREADS;
            v[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (i < n4) v[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, i * 16, 0, 16));
            if (NORM) wt[u] = i < n4 ? reinterpret_cast<const float4*>(w)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < PB; u++) {
            const int i = b0 + tid + u * PK_THREADS;
            if (i < nv4) {
                float4 e = v[u];
                if (NORM) {
                    ss = __builtin_fmaf(e.x, e.x, ss);
                    ss = __builtin_fmaf(e.y, e.y, ss);
                    ss = __builtin_fmaf(e.z, e.z, ss);
                    ss = __builtin_fmaf(e.w, e.w, ss);
                    e = make_float4(e.x * wt[u].x, e.y * wt[u].y, e.z * wt[u].z, e.w * wt[u].w);
                }
                const int k = 4 * i;
                xs[xs_index(k, XS)] = e.x;
                xs[xs_index(k + 1, XS)] = e.y;
                xs[xs_index(k + 2, XS)] = e.z;
                xs[xs_index(k + 3, XS)] = e.w;
            }
        }
    }
    float scale = 1.0f;
    *zero = false;
    if (NORM) {
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        ss += __shfl_xor(ss, 8);
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (lane == 0) ssw[wave] = ss;
    }
    lds_barrier();
    if (NORM) {
        const float tot = (ssw[0] + ssw[1]) + (ssw[2] + ssw[3]);
        const float den = tot / (float)n + 1e-5f;
        *zero = !(den > 0.0f);
        scale = *zero ? 0.0f : 1.0f / sqrtf(den);
    }
    return scale;
}

// ---------------------------------------------------------------- matvec phase

// wave's stream over matrix M: step s (U chunks) of pass p = s / spr
struct PkStream {
    int SK, U, per, cps, c_lo, spr, nsteps, rs, groups, cmax;
    __device__ __forceinline__ int rg_of(int p) const { return (p * (int)gridDim.x + (int)blockIdx.x) * (4 / SK) + rs; }
};

__device__ __forceinline__ PkStream pk_stream(const PMat& M, int wave) {
    PkStream t;
    t.SK = M.SK;
    t.U = M.U;
    t.per = M.per;
    t.cps = M.nchp / M.SK;
    t.c_lo = (wave % M.SK) * t.cps;
    t.rs = wave / M.SK;
    t.spr = (t.cps + M.U - 1) / M.U;
    t.nsteps = M.per * t.spr;
    t.groups = (M.rows + 3) >> 2;
    t.cmax = t.groups * M.nchp + 8 - PK_UMAX;
    return t;
}

__device__ __forceinline__ void pk_load(const PMat& M, const PkStream& t, int s, uint4 (&wb)[PK_UMAX],
                                        uint4 (&db)[PK_UMAX]) {
    const int lane = threadIdx.x & 63, r = lane >> 4;
    const int p = s / t.spr, li = (s - p * t.spr) * t.U;
    const int c = min(min(t.rg_of(p), t.groups) * M.nchp + t.c_lo + li, t.cmax);
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc((void*)M.qs, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc((void*)M.d, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int u = 0; u < PK_UMAX; u++)
        if (u < t.U) {
            wb[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qrs, lane * 16, (c + u) * 1024, 0));
            db[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(drs, r * 16, (c + u) * 64, 0));
        }
}

// the first two steps of this wave's stream over M (issued ahead of a barrier wait)
__device__ __forceinline__ void pk_prefetch(const PMat& M, uint4 (&wA)[PK_UMAX], uint4 (&dA)[PK_UMAX],
                                            uint4 (&wB)[PK_UMAX], uint4 (&dB)[PK_UMAX]) {
    const PkStream t = pk_stream(M, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    if (t.nsteps > 0) pk_load(M, t, 0, wA, dA);
    if (t.nsteps > 1) pk_load(M, t, 1, wB, dB);
}

// one chunk of one lane: acc += d_j * (x0 q0 + x1 q1) over the 8 blocks
__device__ __forceinline__ float pk_chunk_dot(const uint4& w, const uint4& dd, const float* xrow, int cc, float acc) {
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

// y = M x for this workgroup's share of the rows (x staged in xs, the first two steps
// already in A and B), epilogue EPI with coherent activation stores.  With layer_x, the
// RESID epilogue also copies the updated rows there.
template <int EPI>
__device__ __forceinline__ void pk_matvec(const PMat& M, const float* xs, float nscale, bool nzero, float* out,
                                          const MvArgs& a, uint4 (&wA)[PK_UMAX], uint4 (&dA)[PK_UMAX],
                                          uint4 (&wB)[PK_UMAX], uint4 (&dB)[PK_UMAX], float (*red)[4][4],
                                          float& best_v, int& best_i, float* layer_x) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane >> 4, g = lane & 15;
    const PkStream t = pk_stream(M, wv);
    const int ks = wv % t.SK;
    const float* xrow = xs + g * (2 * M.nbp + 4);
    // RESID: the current values of this lane's rows in the first passes, loaded now so the
    // epilogue does not wait a round trip per row
    constexpr int PRE = 4;
    float xres[PRE];
    if (EPI == EPI_RESID && ks == 0 && g == 0) {
#pragma unroll
        for (int p = 0; p < PRE; p++) {
            const int row = t.rg_of(p) * 4 + r;
            xres[p] = (p < t.per && row < M.rows) ? act_ld<true>(out + row) : 0.0f;
        }
    }
    float acc = 0.0f;
    int par = 0;
    auto finish = [&](int p) {
        acc += dpp_f<0x128>(acc);
        acc += dpp_f<0x124>(acc);
        acc += dpp_f<0x4E>(acc);
        acc += dpp_f<0xB1>(acc);  // every lane of the row holds the row's sum
        float y = acc;
        if (t.SK > 1) {
            if (g == 0) red[par][wv][r] = acc;
            lds_barrier();
            if (ks == 0) {
                y = red[par][t.rs * t.SK][r];
                for (int k = 1; k < t.SK; k++) y += red[par][t.rs * t.SK + k][r];
            }
            par ^= 1;
        }
        if (ks == 0) {
            const int rg = t.rg_of(p);
            const int row = rg * 4 + r;
            const bool own = rg < t.groups && g == 0 && row < M.rows;
            y = nzero ? 0.0f : y * nscale;
            if (EPI == EPI_RESID) {
                if (own) {
                    float xo = 0.0f;
#pragma unroll
                    for (int q = 0; q < PRE; q++)
                        if (q == p) xo = xres[q];
                    const float xn = (p < PRE ? xo : act_ld<true>(out + row)) + y;
                    act_st<true>(out + row, xn);
                    if (layer_x) act_st<true>(layer_x + row, xn);
                }
            } else {
                mv_epilogue<EPI, true>(y, row, own, r, M.rows, a, out, best_v, best_i);
            }
        }
        acc = 0.0f;
    };
    auto step = [&](int s, uint4 (&wb)[PK_UMAX], uint4 (&db)[PK_UMAX]) {
        const int p = s / t.spr, ci = (s - p * t.spr) * t.U;
#pragma unroll
        for (int u = 0; u < PK_UMAX; u++)
            if (u < t.U && ci + u < t.cps && t.c_lo + ci + u < M.nch)
                acc = pk_chunk_dot(wb[u], db[u], xrow, t.c_lo + ci + u, acc);
        if (s + 2 < t.nsteps) pk_load(M, t, s + 2, wb, db);
        if (ci + t.U >= t.cps) finish(p);
    };
    for (int s = 0; s < t.nsteps; s += 2) {
        step(s, wA, dA);
        if (s + 1 < t.nsteps) step(s + 1, wB, dB);
    }
}

// ---------------------------------------------------------------- attention phase

// ---------------------------------------------------------------- the kernel

template <int P>
__global__ __launch_bounds__(PK_THREADS, 1) void decode_persist_kernel(PersistArgs A) {
    extern __shared__ __align__(16) float smem[];  // x staging; the attention's tile when it runs
    __shared__ float red[2][4][4];
    __shared__ float ssw[4];
    __shared__ int dead;
    __shared__ int last;
    __shared__ float rowv[16];
    __shared__ int rowi[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) dead = 0;
    const PkSync sync{A.flags, A.err};
    unsigned epoch = 0;
    uint4 wA[PK_UMAX], dA[PK_UMAX], wB[PK_UMAX], dB[PK_UMAX];
    float best_v = -__builtin_inff();
    int best_i = 0x7fffffff;

    MvArgs none;
    AttnArgs at = A.att;
    const int H = A.H;
    pk_prefetch(A.layers[0].qkv, wA, dA, wB, dB);
    __syncthreads();  // dead = 0
    for (int l = 0; l < A.L; l++) {
        const PLayer& Ly = A.layers[l];
        bool nz;
        float sc;
        // ---- QKV: RMSNorm (by linearity), bias, RoPE on q and k
        sc = pk_stage<true>(A.X, H, Ly.qkv.nbp, Ly.rms1, smem, ssw, &nz);
        {
            MvArgs qa;
            qa.aux = Ly.bqkv;
            qa.state = at.state;
            qa.pos0 = at.start_pos;
            qa.cos_t = A.cos_t;
            qa.sin_t = A.sin_t;
            qa.nh = at.nh;
            qa.nkv = at.nkv;
            qa.hd = at.hd;
            pk_matvec<EPI_ROPE>(Ly.qkv, smem, sc, nz, A.qkv, qa, wA, dA, wB, dB, red, best_v, best_i, nullptr);
        }
        pk_arrive(sync, ++epoch);
        pk_wait(sync, epoch, &dead);

        // ---- attention: slice (kvh, s) = workgroup kvh * ns + s; the last slice of a kv head merges
        at.layer = l;
        {
            const int unit = blockIdx.x;
            if (unit < at.nkv * A.ns) {
                const int kvh = unit / A.ns, s = unit - kvh * A.ns;
                SplitLds<P, SPL_GMAX>& L = *reinterpret_cast<SplitLds<P, SPL_GMAX>*>(smem);
                if (attn_slice<P, SPL_GMAX, true>(at, A.ns, A.part, kvh, s, L)) {
                    __builtin_amdgcn_s_waitcnt(0);  // the slice's partial sums are complete
                    __syncthreads();
                    if (tid == 0) {
                        const int pos = at.state ? at.state[0] - 1 : at.start_pos + at.row0;
                        const int nk = pos + 1, chunk = split_chunk(nk, A.ns), live = (nk + chunk - 1) / chunk;
                        const unsigned old =
                            __hip_atomic_fetch_add(A.acnt + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        last = old == (unsigned)(live - 1);
                        if (last) __hip_atomic_store(A.acnt + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    __syncthreads();
                    if (last) {
                        float* ml = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + sizeof(SplitLds<P, SPL_GMAX>));
                        combine_group<P, true>(at, A.ns, A.part, kvh, ml, ml + 2 * SPL_GMAX * 256);
                    }
                }
            }
        }
        pk_arrive(sync, ++epoch);
        pk_prefetch(Ly.o, wA, dA, wB, dB);
        pk_wait(sync, epoch, &dead);

        // ---- O projection + residual
        sc = pk_stage<false>(at.out, at.nh * at.hd, Ly.o.nbp, nullptr, smem, ssw, &nz);
        pk_matvec<EPI_RESID>(Ly.o, smem, sc, nz, A.X, none, wA, dA, wB, dB, red, best_v, best_i, nullptr);
        pk_arrive(sync, ++epoch);
        pk_prefetch(Ly.gu, wA, dA, wB, dB);
        pk_wait(sync, epoch, &dead);

        // ---- gate/up (RMSNorm by linearity) + SwiGLU
        sc = pk_stage<true>(A.X, H, Ly.gu.nbp, Ly.rms2, smem, ssw, &nz);
        pk_matvec<EPI_SWIGLU>(Ly.gu, smem, sc, nz, A.h, none, wA, dA, wB, dB, red, best_v, best_i, nullptr);
        pk_arrive(sync, ++epoch);
        pk_prefetch(Ly.down, wA, dA, wB, dB);
        pk_wait(sync, epoch, &dead);

        // ---- down + residual
        sc = pk_stage<false>(A.h, A.F, Ly.down.nbp, nullptr, smem, ssw, &nz);
        pk_matvec<EPI_RESID>(Ly.down, smem, sc, nz, A.X, none, wA, dA, wB, dB, red, best_v, best_i,
                             A.layer_x ? A.layer_x + (size_t)l * H : nullptr);
        pk_arrive(sync, ++epoch);
        if (l + 1 < A.L)
            pk_prefetch(A.layers[l + 1].qkv, wA, dA, wB, dB);
        else if (A.head)
            pk_prefetch(A.lm, wA, dA, wB, dB);
        pk_wait(sync, epoch, &dead);
    }
    if (!A.head) return;

    // ---- final RMSNorm + lm_head, per-workgroup first maximum, then workgroup 0 picks
    {
        bool nz;
        const float sc = pk_stage<true>(A.X, H, A.lm.nbp, A.final_rms, smem, ssw, &nz);
        pk_matvec<EPI_ARGMAX>(A.lm, smem, sc, nz, A.logits, none, wA, dA, wB, dB, red, best_v, best_i, nullptr);
        if ((lane & 15) == 0) {
            rowv[wave * 4 + (lane >> 4)] = best_v;
            rowi[wave * 4 + (lane >> 4)] = best_i;
        }
        __syncthreads();
        if (tid == 0) {
            float bv = rowv[0];
            int bi = rowi[0];
            for (int i = 1; i < 16; i++)
                if (rowv[i] > bv || (rowv[i] == bv && rowi[i] < bi)) {
                    bv = rowv[i];
                    bi = rowi[i];
                }
            act_st<true>(A.part_val + blockIdx.x, bv);
            __hip_atomic_store(A.part_idx + blockIdx.x, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    pk_arrive(sync, ++epoch);
    pk_wait(sync, epoch, &dead);
    if (blockIdx.x == 0 && wave == 0) {
        // lowest index among equal maxima (the reference's first strict maximum), then
        // ids[len] = pick, len++, and the stop flag on an EOS id (generate.h:57-60, :78-83)
        float bv = -__builtin_inff();
        int bi = 0x7fffffff;
        for (int i = lane; i < (int)gridDim.x; i += 64) {
            const float v = act_ld<true>(A.part_val + i);
            const int ix = __hip_atomic_load(A.part_idx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
            if (bi == 0x7fffffff) bi = 0;
            int* st = A.mstate;
            if (!st[1]) {
                const int len = st[0];
                A.ids[len] = bi;
                st[0] = len + 1;
                for (int e = 0; e < A.neos; e++)
                    if (bi == A.eos[e]) st[1] = 1;
            }
        }
    }
}

// ---------------------------------------------------------------- host side

static int g_pk_cus = 0;

bool persist_supported(int nh, int nkv, int hd) { return g_pk_cus > 0 && attn_split_supported(nh, nkv, hd); }

int persist_workgroups() { return g_pk_cus; }

// slices of the attention: about 128 keys each (a 256-key tile per slice workgroup half
// used at most), at most one workgroup per slice
int persist_slices(int nkv, int max_keys) {
    return std::max(1, std::min(std::min(256, (max_keys + 127) / 128), g_pk_cus / nkv));
}

// LDS of one launch: the largest staged vector (widest input of the layer's matrices and
// the lm_head) or the attention's tile plus its merge arrays
size_t persist_lds_bytes(int max_nbp, int hd) {
    const size_t xs = (size_t)16 * (2 * max_nbp + 4) * sizeof(float);
    const size_t at = (hd == 64 ? sizeof(SplitLds<4, SPL_GMAX>) : sizeof(SplitLds<8, SPL_GMAX>)) + (size_t)3 * SPL_GMAX * 256 * 4;
    return std::max(xs, at);
}

// a matrix's stream plan for the persistent kernel's nwg workgroups: the split SK (1, 2 or
// 4 waves per row group, dividing the stored chunks) and buffer depth U (at most 8, whole
// steps where possible) that give the fewest chunks on the busiest wave
void persist_plan(PMat& M, int nwg) {
    const int groups = (M.rows + 3) / 4;
    long best = -1;
    for (int sk : {1, 2, 4}) {
        if (M.nchp % sk) continue;
        const int cps = M.nchp / sk;
        int u = cps <= PK_UMAX ? cps : 1;
        if (cps > PK_UMAX)
            for (int c = PK_UMAX; c >= 2; c--)
                if (cps % c == 0) {
                    u = c;
                    break;
                }
        if (cps > PK_UMAX && u < 4) u = PK_UMAX;  // no good divisor: full buffers, a partial last step
        const int rpw = 4 / sk;
        const int passes = (groups + rpw - 1) / rpw;
        const int per = (passes + nwg - 1) / nwg;
        const long cost = (long)per * ((cps + u - 1) / u) * u;  // chunk slots the busiest wave streams
        if (best < 0 || cost < best) {
            best = cost;
            M.SK = sk;
            M.U = u;
            M.per = per;
        }
    }
}

void launch_decode_persist(const PersistArgs& A, size_t lds, hipStream_t st) {
    if (A.att.hd == 64)
        hipLaunchKernelGGL(decode_persist_kernel<4>, dim3(g_pk_cus), dim3(PK_THREADS), lds, st, A);
    else
        hipLaunchKernelGGL(decode_persist_kernel<8>, dim3(g_pk_cus), dim3(PK_THREADS), lds, st, A);
}

// one workgroup per CU stays resident with `lds` bytes of dynamic LDS (the launch needs
// every workgroup resident at once)
bool persist_resident(int hd, size_t lds) {
    int occ = 0;
    const hipError_t e =
        hd == 64 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, decode_persist_kernel<4>, PK_THREADS, lds)
                 : hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, decode_persist_kernel<8>, PK_THREADS, lds);
    return e == hipSuccess && occ >= 1 && lds <= 160 * 1024 - 4096;
}

hipError_t persist_init() {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    for (const void* f : {reinterpret_cast<const void*>(&decode_persist_kernel<4>),
                          reinterpret_cast<const void*>(&decode_persist_kernel<8>)})
        if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 4096);
    if (e != hipSuccess) return e;
    g_pk_cus = cus;
    return hipSuccess;
}

}  // namespace jy
