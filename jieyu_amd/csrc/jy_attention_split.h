// jy_attention_split.h — one slice of the split (flash-decoding) decode attention,
// shared by the separate attention kernel and the persistent decode kernel.  See
// jy_attention_split.hip for the arithmetic and what it keeps from attention_q8
// (libs/model_libs/attention/attention_q8.h:38-184, attention/x86/x86_classic.txt:14-73).
#pragma once

#include "jy_layout.h"

namespace jy {

static constexpr int SPL_THREADS = 256;  // one key per thread per tile
static constexpr int SPL_GMAX = 8;       // query heads per kv head this form handles
static constexpr int SPL_MIN_CHUNK = 16;

// keys per slice for nk live keys over ns slices (a multiple of 16), and the slices used
__host__ __device__ __forceinline__ int split_chunk(int nk, int ns) {
    int c = (nk + ns - 1) / ns;
    c = (c + SPL_MIN_CHUNK - 1) / SPL_MIN_CHUNK * SPL_MIN_CHUNK;
    return c < SPL_MIN_CHUNK ? SPL_MIN_CHUNK : c;
}

__device__ __forceinline__ float wave_sum64(float v) {
    // fixed butterfly order: the same bits whatever the launch
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// e^x from the hardware exp2 (v_exp_f32): about 1 ulp plus the rounding of x*log2(e),
// a relative error under 1e-6 for the |x| <= 20 that carry weight here
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// LDS of one slice (a struct so that a kernel can place it in static or dynamic LDS)
template <int P>
struct SplitLds {
    static constexpr int HD = P * 16, NW = SPL_THREADS / 64, KS = SPL_THREADS / HD;
    int8_t q8[SPL_GMAX][HD] __attribute__((aligned(16)));
    int8_t vt[SPL_THREADS][HD + 16] __attribute__((aligned(16)));  // V tile, rows padded
    int8_t knew[HD] __attribute__((aligned(16)));
    int8_t vnew[HD] __attribute__((aligned(16)));
    float qsc[SPL_GMAX];
    float pw[SPL_GMAX][SPL_THREADS];  // e_j * vs_j of the tile
    float redm[NW][SPL_GMAX], reds[NW][SPL_GMAX];
    float kvs_new[2];
    float accs[KS - 1][SPL_GMAX][HD];
};

// One (kv head, slice of keys) unit of the split attention, by the whole workgroup
// (SPL_THREADS threads): writes the slice's (o[hd], max, sum) for each query head of the
// group to part.  Returns false (having done nothing) for a slice past the live length.
// P = hd / 16: 16-byte pieces per key row.
template <int P, bool COH>
__device__ __forceinline__ bool attn_slice(const AttnArgs& a, int ns, float* __restrict__ part, int kvh, int s,
                                           SplitLds<P>& L) {
    constexpr int HD = P * 16;
    constexpr int NW = SPL_THREADS / 64;
    constexpr int KS = SPL_THREADS / HD;  // key subsets of the p.v phase (4 for hd 64, 2 for hd 128)
    auto& q8 = L.q8;
    auto& qsc = L.qsc;
    auto& vt = L.vt;
    auto& pw = L.pw;
    auto& redm = L.redm;
    auto& reds = L.reds;
    auto& knew = L.knew;
    auto& vnew = L.vnew;
    auto& kvs_new = L.kvs_new;
    auto& accs = L.accs;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nh = a.nh, nkv = a.nkv, G = nh / nkv;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + a.row0;
    const int nk = pos + 1;
    const int chunk = split_chunk(nk, ns);
    const int j0 = s * chunk;
    if (j0 >= nk) return false;  // whole workgroup: a slice past the live length
    const int j1 = min(nk, j0 + chunk);
    const bool holds_new = j1 == nk;  // this slice ends at the token's own position
    const size_t head = (size_t)a.layer * nkv + kvh;
    int8_t* K = a.kv.k + head * a.kv.max_seq * HD;
    int8_t* V = a.kv.v + head * a.kv.max_seq * HD;
    float* KSc = a.kv.ks + head * a.kv.max_seq;
    float* VSc = a.kv.vs + head * a.kv.max_seq;
    const float* row = a.qkv;  // one token row: q [nh*hd] | k [nkv*hd] | v [nkv*hd]

    // every load that depends only on the position goes out first: this tile's K and V
    // rows and scales (the token's own key comes from the workgroup's copy instead) and
    // the fp32 vectors this wave quantises (items wave, wave+4, wave+8: the group's query
    // heads, then with the new position its k and v)
    auto load_row = [&](const int8_t* base, int j, int4* r) {
#pragma unroll
        for (int c = 0; c < P; c++) r[c] = *reinterpret_cast<const int4*>(base + (size_t)j * HD + 16 * c);
    };
    int4 kr[P], vr[P];
    float ksj = 0.0f, vsj = 0.0f;
    {
        const int j = j0 + tid;
        if (j < j1 && j != pos) {
            load_row(K, j, kr);
            load_row(V, j, vr);
            ksj = KSc[j];
            vsj = VSc[j];
        }
    }
    const int nitems = G + (holds_new ? 2 : 0);
    constexpr int PER = HD / 64;  // elements per lane of one vector
    float qv[3][PER];
#pragma unroll
    for (int t = 0; t < 3; t++) {
        const int i = wave + NW * t;
        if (i < nitems) {
            const float* src = i < G ? row + (size_t)(kvh * G + i) * HD
                                     : row + (size_t)((i == G ? nh : nh + nkv) + kvh) * HD;
#pragma unroll
            for (int c = 0; c < PER; c++) qv[t][c] = act_ld<COH>(src + lane + 64 * c);
        }
    }
#pragma unroll
    for (int t = 0; t < 3; t++) {
        const int i = wave + NW * t;
        if (i < nitems) {
            float amax = 0.0f;
#pragma unroll
            for (int c = 0; c < PER; c++) amax = fmaxf(amax, fabsf(qv[t][c]));
            amax = wave_max64(amax);
            const float inv = quant_inv(amax);
            int8_t* dst = i < G ? q8[i] : (i == G ? knew : vnew);
#pragma unroll
            for (int c = 0; c < PER; c++) dst[lane + 64 * c] = quant_i8(qv[t][c], inv);
            if (lane == 0) {
                if (i < G)
                    qsc[i] = quant_scale(amax);
                else
                    kvs_new[i == G ? 0 : 1] = quant_scale(amax);
            }
        }
    }
    __syncthreads();
    if (holds_new) {
        // kv_pack_q8 of the new position: appended by the one workgroup that holds it
        for (int d = tid; d < HD; d += SPL_THREADS) {
            K[(size_t)pos * HD + d] = knew[d];
            V[(size_t)pos * HD + d] = vnew[d];
        }
        if (tid == 0) {
            KSc[pos] = kvs_new[0];
            VSc[pos] = kvs_new[1];
        }
    }

    const float scale = 1.0f / sqrtf((float)HD);
    float m_run[SPL_GMAX], l_run[SPL_GMAX], acc[SPL_GMAX];
#pragma unroll
    for (int g = 0; g < SPL_GMAX; g++) {
        m_run[g] = -__builtin_inff();
        l_run[g] = 0.0f;
        acc[g] = 0.0f;
    }
    // p.v mapping: thread = (output dim d, key subset kq)
    const int d = tid % HD, kq = tid / HD;

    for (int t0 = j0; t0 < j1; t0 += SPL_THREADS) {
        const int j = t0 + tid;
        const bool live = j < j1;
        if (live && j == pos) {
#pragma unroll
            for (int c = 0; c < P; c++) {
                kr[c] = *reinterpret_cast<const int4*>(knew + 16 * c);
                vr[c] = *reinterpret_cast<const int4*>(vnew + 16 * c);
            }
            ksj = kvs_new[0];
            vsj = kvs_new[1];
        }
        // V row into the tile (dim-major reads later)
#pragma unroll
        for (int c = 0; c < P; c++) *reinterpret_cast<int4*>(&vt[tid][16 * c]) = live ? vr[c] : make_int4(0, 0, 0, 0);
        // exact int32 dots against every query head of the group
        float sc[SPL_GMAX];
#pragma unroll
        for (int g = 0; g < SPL_GMAX; g++) {
            sc[g] = -__builtin_inff();
            if (g < G && live) {
                int dot = 0;
#pragma unroll
                for (int c = 0; c < P; c++) {
                    const int4 q4 = *reinterpret_cast<const int4*>(&q8[g][16 * c]);
                    dot = __builtin_amdgcn_sdot4(q4.x, kr[c].x, dot, false);
                    dot = __builtin_amdgcn_sdot4(q4.y, kr[c].y, dot, false);
                    dot = __builtin_amdgcn_sdot4(q4.z, kr[c].z, dot, false);
                    dot = __builtin_amdgcn_sdot4(q4.w, kr[c].w, dot, false);
                }
                sc[g] = (float)dot * ((ksj * qsc[g]) * scale);
            }
        }
        // the next tile's rows are independent of this one's math: request them now
        const int jn = j + SPL_THREADS;
        const bool next = jn < j1 && jn != pos;
        if (next) {
            load_row(K, jn, kr);
            load_row(V, jn, vr);
        }
        const float ks_next = next ? KSc[jn] : 0.0f;
        const float vs_next = next ? VSc[jn] : 0.0f;
        // tile maximum per head: waves, then the workgroup
#pragma unroll
        for (int g = 0; g < SPL_GMAX; g++)
            if (g < G) {
                const float mw = wave_max64(sc[g]);
                if (lane == 0) redm[wave][g] = mw;
            }
        __syncthreads();
        // running maximum, the rescale of what came before, this tile's weights and sums
        float e[SPL_GMAX];
#pragma unroll
        for (int g = 0; g < SPL_GMAX; g++)
            if (g < G) {
                float mt = redm[0][g];
#pragma unroll
                for (int w = 1; w < NW; w++) mt = fmaxf(mt, redm[w][g]);
                const float mn = fmaxf(m_run[g], mt);
                const float al = m_run[g] == -__builtin_inff() ? 0.0f : exp_hw(m_run[g] - mn);
                m_run[g] = mn;
                e[g] = live ? exp_hw(sc[g] - mn) : 0.0f;
                pw[g][tid] = e[g] * vsj;
                l_run[g] *= al;
                acc[g] *= al;
                const float sw = wave_sum64(e[g]);
                if (lane == 0) reds[wave][g] = sw;
            }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < SPL_GMAX; g++)
            if (g < G) {
                float st = reds[0][g];
#pragma unroll
                for (int w = 1; w < NW; w++) st += reds[w][g];
                l_run[g] += st;
            }
        // o[g][d] += sum over this subset's keys (every KS-th key of the tile) of (e * vs) * v
        const int tn = min(SPL_THREADS, j1 - t0);
        for (int t = kq; t < tn; t += KS) {
            const float vv = (float)vt[t][d];
#pragma unroll
            for (int g = 0; g < SPL_GMAX; g++)
                if (g < G) acc[g] = __builtin_fmaf(pw[g][t], vv, acc[g]);
        }
        ksj = ks_next;
        vsj = vs_next;
        if (t0 + SPL_THREADS < j1) __syncthreads();  // vt / pw / red are rewritten by the next tile
    }

    // the key subsets' partial sums, in subset order
    if (kq > 0) {
#pragma unroll
        for (int g = 0; g < SPL_GMAX; g++)
            if (g < G) accs[kq - 1][g][d] = acc[g];
    }
    __syncthreads();
    if (kq == 0) {
#pragma unroll
        for (int q = 1; q < KS; q++)
#pragma unroll
            for (int g = 0; g < SPL_GMAX; g++)
                if (g < G) acc[g] += accs[q - 1][g][d];
        const int W = HD + 2;
#pragma unroll
        for (int g = 0; g < SPL_GMAX; g++)
            if (g < G) {
                float* o = part + ((size_t)(kvh * G + g) * ns + s) * W;
                act_st<COH>(o + d, acc[g]);
                if (d == 0) {
                    act_st<COH>(o + HD, m_run[g]);
                    act_st<COH>(o + HD + 1, l_run[g]);
                }
            }
    }
    return true;
}

}  // namespace jy
