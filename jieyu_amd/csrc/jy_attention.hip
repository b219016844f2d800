// jy_attention.hip — GQA attention over the int8 KV cache, bit-exact with
// attention_q8 (libs/model_libs/attention/attention_q8.h:20-37, :38-184 and
// attention/x86/x86_classic.txt:10-73):
//   Q -> int8 per head (absmax, lrintf); exact int32 q.k for every key j <= p;
//   score_j = (float)dot * ((ks_j * qsc) * (1/sqrtf(hd))); strict max from -1e30;
//   e_j = expf(score_j - max); sum += e_j in ascending j; p_j = e_j * (1/sum);
//   o[d] = fma(p_j * vs_j, (float)v8[j][d], o[d]) in ascending j.
//
// One workgroup per (query head, token row, slice of 32 output dims).  The scores
// are parallel; the softmax sum and the output components are the reference's
// ascending chains, run from LDS: the sum on one lane while the other waves stage
// this slice of V (as fp16, exact for int8, so each chain step is one v_fma_mix),
// then one lane per output dim.  In the fused decode form the kernel also quantises
// the token's q, k and v itself and the first head of each GQA group appends k/v to
// the cache (kv_pack_q8 of the new position).
#include "jy_layout.h"

namespace jy {

static constexpr int ATT_THREADS = 256;
static constexpr int ATT_ECAP = 4096;   // scores kept in LDS up to this many keys
static constexpr int ATT_WIN = 2048;    // window of the sum chain beyond that

__device__ __forceinline__ float att_block_max(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

// absmax int8 quantisation of one head vector by one wave (kv_pack_q8)
__device__ __forceinline__ void att_quant(const float* src, int hd, int8_t* dst, float* scale_out) {
    const int lane = threadIdx.x & 63;
    float amax = 0.0f;
    for (int d = lane; d < hd; d += 64) amax = fmaxf(amax, fabsf(src[d]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const float inv = quant_inv(amax);
    for (int d = lane; d < hd; d += 64) dst[d] = quant_i8(src[d], inv);
    if (lane == 0) *scale_out = quant_scale(amax);
}

// The two sequential chains of the reference softmax/PV, with their LDS operands
// fetched 16 steps ahead into registers so each step is one dependent VALU op.
__device__ __forceinline__ float chain_sum(const float* e, int n, float sum) {
    int j = 0;
    if (n >= 16) {
        const float4* e4 = reinterpret_cast<const float4*>(e);
        float4 c0 = e4[0], c1 = e4[1], c2 = e4[2], c3 = e4[3];
        for (; j + 32 <= n; j += 16) {
            const float4 n0 = e4[(j >> 2) + 4], n1 = e4[(j >> 2) + 5], n2 = e4[(j >> 2) + 6], n3 = e4[(j >> 2) + 7];
            sum += c0.x; sum += c0.y; sum += c0.z; sum += c0.w;
            sum += c1.x; sum += c1.y; sum += c1.z; sum += c1.w;
            sum += c2.x; sum += c2.y; sum += c2.z; sum += c2.w;
            sum += c3.x; sum += c3.y; sum += c3.z; sum += c3.w;
            c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        }
        sum += c0.x; sum += c0.y; sum += c0.z; sum += c0.w;
        sum += c1.x; sum += c1.y; sum += c1.z; sum += c1.w;
        sum += c2.x; sum += c2.y; sum += c2.z; sum += c2.w;
        sum += c3.x; sum += c3.y; sum += c3.z; sum += c3.w;
        j += 16;
    }
    for (; j < n; j++) sum += e[j];
    return sum;
}

__device__ __forceinline__ float hx(uint32_t w, int hi) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? (w >> 16) : w));
}

// o = fma(p_j, v_j, o) for j ascending; v as fp16 (exact int8), one v_fma_mix per step
__device__ __forceinline__ float chain_pv(const float* P, const _Float16* vr, float o, int n) {
    int j = 0;
    if (n >= 16) {
        const float4* p4 = reinterpret_cast<const float4*>(P);
        const uint4* v4 = reinterpret_cast<const uint4*>(vr);
        float4 a0 = p4[0], a1 = p4[1], a2 = p4[2], a3 = p4[3];
        uint4 b0 = v4[0], b1 = v4[1];
        auto steps = [&](const float4& q0, const float4& q1, const float4& q2, const float4& q3, const uint4& u0,
                         const uint4& u1) {
            o = __builtin_fmaf(q0.x, hx(u0.x, 0), o); o = __builtin_fmaf(q0.y, hx(u0.x, 1), o);
            o = __builtin_fmaf(q0.z, hx(u0.y, 0), o); o = __builtin_fmaf(q0.w, hx(u0.y, 1), o);
            o = __builtin_fmaf(q1.x, hx(u0.z, 0), o); o = __builtin_fmaf(q1.y, hx(u0.z, 1), o);
            o = __builtin_fmaf(q1.z, hx(u0.w, 0), o); o = __builtin_fmaf(q1.w, hx(u0.w, 1), o);
            o = __builtin_fmaf(q2.x, hx(u1.x, 0), o); o = __builtin_fmaf(q2.y, hx(u1.x, 1), o);
            o = __builtin_fmaf(q2.z, hx(u1.y, 0), o); o = __builtin_fmaf(q2.w, hx(u1.y, 1), o);
            o = __builtin_fmaf(q3.x, hx(u1.z, 0), o); o = __builtin_fmaf(q3.y, hx(u1.z, 1), o);
            o = __builtin_fmaf(q3.z, hx(u1.w, 0), o); o = __builtin_fmaf(q3.w, hx(u1.w, 1), o);
        };
        for (; j + 32 <= n; j += 16) {
            const float4 n0 = p4[(j >> 2) + 4], n1 = p4[(j >> 2) + 5], n2 = p4[(j >> 2) + 6], n3 = p4[(j >> 2) + 7];
            const uint4 m0 = v4[(j >> 3) + 2], m1 = v4[(j >> 3) + 3];
            steps(a0, a1, a2, a3, b0, b1);
            a0 = n0; a1 = n1; a2 = n2; a3 = n3; b0 = m0; b1 = m1;
        }
        steps(a0, a1, a2, a3, b0, b1);
        j += 16;
    }
    for (; j < n; j++) o = __builtin_fmaf(P[j], (float)vr[j], o);
    return o;
}

__global__ __launch_bounds__(ATT_THREADS) void attention_kernel(AttnArgs a, int ds, int vcap) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ __align__(16) int8_t qv8[256];
    __shared__ __align__(16) int8_t kloc[256];
    __shared__ __align__(16) int8_t vloc[256];
    __shared__ float sc3[3];  // qsc, kscale, vscale
    __shared__ float red[8];
    __shared__ float s_inv;
    float* E = reinterpret_cast<float*>(smem);                                   // [ATT_ECAP]
    _Float16* VH = reinterpret_cast<_Float16*>(smem + ATT_ECAP * sizeof(float));  // [ds][vcap]

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = blockIdx.x, rr = blockIdx.y, slice = blockIdx.z;
    const int r = a.row0 + rr;
    const int hd = a.hd, nh = a.nh, nkv = a.nkv, group = nh / nkv, kvh = h / group;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + r;
    const int nk = pos + 1;
    const int d0 = slice * ds;
    const size_t head = (size_t)a.layer * nkv + kvh;
    const int8_t* K = a.kv.k + head * a.kv.max_seq * hd;
    const int8_t* V = a.kv.v + head * a.kv.max_seq * hd;
    const float* KS = a.kv.ks + head * a.kv.max_seq;
    const float* VS = a.kv.vs + head * a.kv.max_seq;
    const bool fused = a.fused;
    const bool long_ctx = nk > ATT_ECAP;
    float* G = a.scratch + ((size_t)rr * nh + h) * a.max_keys;  // long contexts: scores in HBM

    // ---- this token's q (and, fused, k and v) as int8
    if (fused) {
        const float* row = a.qkv + (size_t)rr * (nh + 2 * nkv) * hd;
        if (wave == 0) att_quant(row + (size_t)h * hd, hd, qv8, &sc3[0]);
        if (wave == 1) att_quant(row + (size_t)(nh + kvh) * hd, hd, kloc, &sc3[1]);
        if (wave == 2) att_quant(row + (size_t)(nh + nkv + kvh) * hd, hd, vloc, &sc3[2]);
    } else if (wave == 0) {
        const int8_t* q = a.q8 + ((size_t)r * nh + h) * hd;
        for (int d = lane; d < hd; d += 64) qv8[d] = q[d];
        if (lane == 0) sc3[0] = a.qsc[(size_t)r * nh + h];
    }
    __syncthreads();
    if (fused && slice == 0 && h % group == 0) {  // the group's first head appends k/v
        const size_t slot = head * a.kv.max_seq + pos;
        for (int d = tid; d < hd; d += blockDim.x) {
            a.kv.k[slot * hd + d] = kloc[d];
            a.kv.v[slot * hd + d] = vloc[d];
        }
        if (tid == 0) {
            a.kv.ks[slot] = sc3[1];
            a.kv.vs[slot] = sc3[2];
        }
    }

    // ---- scores
    const float qs = sc3[0];
    const float scale = 1.0f / sqrtf((float)hd);
    const int nwords = hd >> 2;
    const int32_t* q32 = reinterpret_cast<const int32_t*>(qv8);
    const bool vec = (hd & 15) == 0;
    int4 qw4[16];  // the int8 query as 16-byte words (hd <= 256), loop-invariant
#pragma unroll
    for (int i = 0; i < 16; i++)
        if (vec && i < (hd >> 4)) qw4[i] = reinterpret_cast<const int4*>(qv8)[i];
    float lmax = -1e30f;
    auto score_of = [&](int j, int dot) {
        const bool here = fused && j == pos;
        const float ksj = here ? sc3[1] : KS[j];
        const float sv = (float)dot * ((ksj * qs) * scale);
        if (long_ctx)
            G[j] = sv;
        else
            E[j] = sv;
        lmax = fmaxf(lmax, sv);
    };
    // exact int32 q.k (|q|,|k| <= 127); two keys per thread per pass keep 32 loads in flight
    for (int j = tid; j < nk; j += 2 * blockDim.x) {
        const int j2 = j + blockDim.x;
        const bool here = fused && j == pos, here2 = fused && j2 == pos;
        if (vec && !here && !here2 && j2 < nk) {
            const int4* k4a = reinterpret_cast<const int4*>(K + (size_t)j * hd);
            const int4* k4b = reinterpret_cast<const int4*>(K + (size_t)j2 * hd);
            int4 ka[16], kb[16];
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (i < (hd >> 4)) {
                    ka[i] = k4a[i];
                    kb[i] = k4b[i];
                }
            int da = 0, db = 0;
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (i < (hd >> 4)) {
                    da = __builtin_amdgcn_sdot4(qw4[i].x, ka[i].x, da, false);
                    da = __builtin_amdgcn_sdot4(qw4[i].y, ka[i].y, da, false);
                    da = __builtin_amdgcn_sdot4(qw4[i].z, ka[i].z, da, false);
                    da = __builtin_amdgcn_sdot4(qw4[i].w, ka[i].w, da, false);
                    db = __builtin_amdgcn_sdot4(qw4[i].x, kb[i].x, db, false);
                    db = __builtin_amdgcn_sdot4(qw4[i].y, kb[i].y, db, false);
                    db = __builtin_amdgcn_sdot4(qw4[i].z, kb[i].z, db, false);
                    db = __builtin_amdgcn_sdot4(qw4[i].w, kb[i].w, db, false);
                }
            score_of(j, da);
            score_of(j2, db);
            continue;
        }
        for (int jj = j; jj <= j2 && jj < nk; jj += blockDim.x) {
            const bool h1 = fused && jj == pos;
            const int32_t* k32 = h1 ? reinterpret_cast<const int32_t*>(kloc)
                                    : reinterpret_cast<const int32_t*>(K + (size_t)jj * hd);
            int dot = 0;
            for (int i = 0; i < nwords; i++) dot = __builtin_amdgcn_sdot4(q32[i], k32[i], dot, false);
            score_of(jj, dot);
        }
    }
    const float mx = att_block_max(lmax, red);
    for (int j = tid; j < nk; j += blockDim.x) {
        if (long_ctx)
            G[j] = expf_libm(G[j] - mx);
        else
            E[j] = expf_libm(E[j] - mx);
    }
    __syncthreads();

    // ---- sum chain (wave 0, lane 0) while waves 1.. stage V chunk 0
    const int nstage_thr = blockDim.x - 64;
    auto stage_v = [&](int j0, int cnt) {  // V[j0 .. j0+cnt)[d0 .. d0+ds) -> VH (fp16, [d][j])
        const int t = tid - 64;
        if ((ds & 15) == 0) {  // 16-byte pieces, eight in flight per thread
            const int pieces = ds >> 4, total = cnt * pieces;
            for (int base = t; base < total; base += 8 * nstage_thr) {
                uint4 w[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int e = base + u * nstage_thr;
                    if (e < total) {
                        const int jj = e / pieces, pc = e - jj * pieces, j = j0 + jj;
                        w[u] = (fused && j == pos) ? *reinterpret_cast<const uint4*>(vloc + d0 + pc * 16)
                                                   : *reinterpret_cast<const uint4*>(V + (size_t)j * hd + d0 + pc * 16);
                    }
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int e = base + u * nstage_thr;
                    if (e < total) {
                        const int jj = e / pieces, pc = e - jj * pieces;
                        const uint32_t wv[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
                        for (int b = 0; b < 16; b++)
                            VH[(size_t)(pc * 16 + b) * vcap + jj] = (_Float16)(int8_t)(wv[b >> 2] >> (8 * (b & 3)));
                    }
                }
            }
        } else {  // 4-byte pieces (head dims that are not a multiple of 16)
            const int pieces = ds >> 2, total = cnt * pieces;
            for (int e = t; e < total; e += nstage_thr) {
                const int jj = e / pieces, pc = e - jj * pieces, j = j0 + jj;
                const uint32_t w = (fused && j == pos) ? *reinterpret_cast<const uint32_t*>(vloc + d0 + pc * 4)
                                                       : *reinterpret_cast<const uint32_t*>(V + (size_t)j * hd + d0 + pc * 4);
#pragma unroll
                for (int b = 0; b < 4; b++) VH[(size_t)(pc * 4 + b) * vcap + jj] = (_Float16)(int8_t)(w >> (8 * b));
            }
        }
    };
    const int c0 = nk < vcap ? nk : vcap;
    if (!long_ctx) {
        if (tid == 0) s_inv = 1.0f / chain_sum(E, nk, 0.0f);
        if (wave > 0) stage_v(0, c0);
        __syncthreads();
    } else {
        // windows of the HBM score array through LDS (E doubles as two windows)
        float sum = 0.0f;
        for (int w0 = 0; w0 < nk; w0 += 2 * ATT_WIN) {
            for (int b = 0; b < 2; b++) {
                const int ws = w0 + b * ATT_WIN;
                for (int j = tid; j < ATT_WIN && ws + j < nk; j += blockDim.x) E[b * ATT_WIN + j] = G[ws + j];
            }
            __syncthreads();
            if (tid == 0) {
                const int cnt = min(2 * ATT_WIN, nk - w0);
                sum = chain_sum(E, cnt, sum);
            }
            __syncthreads();
        }
        if (tid == 0) s_inv = 1.0f / sum;
        if (wave > 0) stage_v(0, c0);
        __syncthreads();
    }
    const float inv = s_inv;
    // p_j * vs_j (the reference scales by 1/sum in place, then multiplies by vs_j)
    for (int base = tid; base < nk; base += 8 * blockDim.x) {
        float vsv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = base + u * blockDim.x;
            if (j < nk) vsv[u] = (fused && j == pos) ? sc3[2] : VS[j];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = base + u * blockDim.x;
            if (j < nk) {
                if (long_ctx)
                    G[j] = (G[j] * inv) * vsv[u];
                else
                    E[j] = (E[j] * inv) * vsv[u];
            }
        }
    }
    __syncthreads();

    // ---- output chains, one lane per dim of this slice
    float o = 0.0f;
    for (int cstart = 0; cstart < nk; cstart += vcap) {
        const int cnt = min(vcap, nk - cstart);
        if (cstart > 0) {
            __syncthreads();
            if (wave > 0) stage_v(cstart, cnt);
            if (long_ctx)
                for (int j = tid; j < cnt && j < ATT_ECAP; j += blockDim.x) E[j] = G[cstart + j];
            __syncthreads();
        } else if (long_ctx) {
            for (int j = tid; j < cnt && j < ATT_ECAP; j += blockDim.x) E[j] = G[j];
            __syncthreads();
        }
        if (tid < ds) o = chain_pv(long_ctx ? E : E + cstart, VH + (size_t)tid * vcap, o, cnt);
    }
    if (tid < ds) a.out[((size_t)r * nh + h) * hd + d0 + tid] = o;
}

static int g_att_lds_max = 0;

static void att_shape(int hd, int* ds, int* vcap) {
    *ds = (hd % 32 == 0) ? 32 : hd;
    // fp16 V slice: ds * vcap * 2 bytes next to the ATT_ECAP score floats
    const int budget = (g_att_lds_max > 0 ? g_att_lds_max : 65536) - ATT_ECAP * 4 - 2048;
    int v = 2048;
    while (v > 64 && (size_t)(*ds) * v * 2 > (size_t)budget) v >>= 1;
    *vcap = v;
}

void launch_attention(const AttnArgs& a, hipStream_t st) {
    int ds, vcap;
    att_shape(a.hd, &ds, &vcap);
    const size_t lds = (size_t)ATT_ECAP * 4 + (size_t)ds * vcap * 2;
    hipLaunchKernelGGL(attention_kernel, dim3(a.nh, a.nrows, a.hd / ds), dim3(ATT_THREADS), lds, st, a, ds, vcap);
}

hipError_t matvec_init();

hipError_t kernels_init() {
    int dev = 0, mx = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return e;
    g_att_lds_max = mx;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, mx - 2048);
    if (e != hipSuccess) return e;
    return matvec_init();
}

}  // namespace jy
