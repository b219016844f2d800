// jy_attention_split.h — one slice of the split (flash-decoding) decode attention,
// shared by the separate attention kernel and the persistent decode kernel.  See
// jy_attention_split.hip for the arithmetic and what it keeps from attention_q8
// (libs/model_libs/attention/attention_q8.h:38-184, attention/x86/x86_classic.txt:14-73).
#pragma once

#include "jy_layout.h"

namespace jy {

static constexpr int SPL_THREADS = 256;  // one key per thread per tile
static constexpr int SPL_GMAX = 8;       // query heads per kv head this form handles

// query heads per kv head as a kernel instance computes them: 1, 2, 4 or 8 (the heads
// past the real count carry a zero query and are never written out)
__host__ __device__ constexpr int split_heads(int G) { return G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8; }

// sum over the 64 lanes of a wave, in every lane, in a fixed order: rows of 16 by DPP,
// then the four row sums
__device__ __forceinline__ float wave_sum64(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm 1,0,3,2
    v += dpp_f<0x4E>(v);   // quad_perm 2,3,0,1
    v += dpp_f<0x124>(v);  // row_ror 4
    v += dpp_f<0x128>(v);  // row_ror 8
    return (read_lane(v, 0) + read_lane(v, 16)) + (read_lane(v, 32) + read_lane(v, 48));
}


// Sum of each group of LP adjacent lanes (LP 4 or 8) into the group's last lane, by DPP row
// shifts within rows of 16 lanes (exact: integer adds)
template <int LP>
__device__ __forceinline__ int piece_sum_last(int d) {
    d += __builtin_amdgcn_update_dpp(0, d, 0x111, 0xf, 0xf, true);  // row_shr 1
    d += __builtin_amdgcn_update_dpp(0, d, 0x112, 0xf, 0xf, true);  // row_shr 2
    if (LP > 4) d += __builtin_amdgcn_update_dpp(0, d, 0x114, 0xf, 0xf, true);  // row_shr 4
    return d;
}

// LDS of one slice (a struct so that a kernel can place it in static or dynamic LDS).
// The tile arrays and the final per-subset sums of p.v share their space.
template <int P, int GT>
struct SplitLds {
    static constexpr int HD = P * 16, NW = SPL_THREADS / 64;
    static constexpr int DG = HD / 4, NKS = SPL_THREADS / DG;  // p.v: 4 dims per thread, key subsets
    struct Tile {
        int8_t vt[SPL_THREADS][HD];  // V rows of the tile
        int dots[SPL_THREADS][GT];   // int32 q.k of each key and query head
        float pw[GT][SPL_THREADS];   // e_j * vs_j
    };
    union {
        Tile t;
        float accs[NKS][GT][HD];  // after the last tile: each key subset's o
    } u __attribute__((aligned(16)));
    int8_t q8[GT][HD] __attribute__((aligned(16)));
    int8_t knew[HD] __attribute__((aligned(16)));
    int8_t vnew[HD] __attribute__((aligned(16)));
    float qsc[GT];
    float redm[NW][GT], reds[NW][GT];
    float kvs_new[2];
};

// One (kv head, slice of keys) unit of the split attention, by the whole workgroup
// (SPL_THREADS threads): writes the slice's (o[hd], max, sum) for each query head of the
// group to part.  Returns false (having done nothing) for a slice past the live length.
// P = hd / 16: 16-byte pieces per key row; GT = split_heads(nh / nkv).
// Decode (a.fused): one token row; the workgroup quantises q, and with the slice that
// holds the token's position its k and v, which it appends to the cache.  Prompt rows
// (!a.fused): row `prow` of the launch at position start_pos + row0 + prow, q8 / qsc from
// the RoPE + packing pass and every key already in the cache; with part == nullptr the
// slice is the row's whole key range and o / sum goes straight to a.out.
//
// Per tile of 256 keys:
//  1. the K and V rows arrive as 16-byte pieces, P adjacent lanes per key (every load
//     instruction of a wave reads 64 / P whole rows, contiguous); each lane takes the
//     int32 dot of its piece with each query head's piece, and a DPP sum puts the key's
//     dot in the group's last lane, which stores it; the V pieces go to the LDS tile;
//  2. one key per thread: scores, the tile maximum per head, the weights and their sums;
//  3. p.v: each thread accumulates 4 output dims over every NKS-th quad of keys.
template <int P, int GT, bool COH>
__device__ __forceinline__ bool attn_slice(const AttnArgs& a, int ns, float* __restrict__ part, int kvh, int s,
                                           SplitLds<P, GT>& L, int prow = 0) {
    using Lds = SplitLds<P, GT>;
    constexpr int HD = Lds::HD, NW = Lds::NW, DG = Lds::DG, NKS = Lds::NKS;
    auto& vt = L.u.t.vt;
    auto& dots = L.u.t.dots;
    auto& pw = L.u.t.pw;
    auto& accs = L.u.accs;
    auto& q8 = L.q8;
    auto& qsc = L.qsc;
    auto& redm = L.redm;
    auto& reds = L.reds;
    auto& knew = L.knew;
    auto& vnew = L.vnew;
    auto& kvs_new = L.kvs_new;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nh = a.nh, nkv = a.nkv, G = nh / nkv;  // G <= GT
    const bool fused = a.fused;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + a.row0 + prow;
    const int nk = pos + 1;
    const int chunk = split_chunk(nk, ns);
    const int j0 = s * chunk;
    if (j0 >= nk) return false;  // whole workgroup: a slice past the live length
    const int j1 = min(nk, j0 + chunk);
    const bool holds_new = fused && j1 == nk;  // this slice ends at the token's own position
    // the key taken from the workgroup's copy, only where it lies in the slice (a tile of the
    // slice before may reach past its end onto it, where it is masked like any other)
    const int own = holds_new ? pos : -1;
    const size_t head = (size_t)a.layer * nkv + kvh;
    int8_t* K = a.kv.k + head * a.kv.max_seq * HD;
    int8_t* V = a.kv.v + head * a.kv.max_seq * HD;
    float* KSc = a.kv.ks + head * a.kv.max_seq;
    float* VSc = a.kv.vs + head * a.kv.max_seq;
    const float* row = a.qkv;  // one token row: q [nh*hd] | k [nkv*hd] | v [nkv*hd]

    // every load that depends only on the position goes out first: this tile's K and V
    // pieces (load round u: keys u*KPR .. u*KPR+KPR-1 of the tile, this thread holding
    // piece pc of key u*KPR + kr) and the scales of this thread's key (the token's own
    // key comes from the workgroup's copy instead), then the fp32 vectors this wave
    // quantises (items wave, wave+4, wave+8: the group's query heads, then with the new
    // position its k and v)
    constexpr int KPR = SPL_THREADS / P;
    const int pc = tid % P, kr = tid / P;
    int4 kp[P], vp[P];
#pragma unroll
    for (int u = 0; u < P; u++) kp[u] = vp[u] = make_int4(0, 0, 0, 0);
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int u = 0; u < P; u++) {
            const int j = t0 + u * KPR + kr;
            if (j < j1 && j != own) {
                kp[u] = *reinterpret_cast<const int4*>(K + (size_t)j * HD + 16 * pc);
                vp[u] = *reinterpret_cast<const int4*>(V + (size_t)j * HD + 16 * pc);
            }
        }
    };
    load_tile(j0);
    float ksj = 0.0f, vsj = 0.0f;  // the scales of key t0 + tid, this thread's in the softmax
    {
        const int j = j0 + tid;
        if (j < j1 && j != own) {
            ksj = KSc[j];
            vsj = VSc[j];
        }
    }
    const int nitems = fused ? G + (holds_new ? 2 : 0) : 0;
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
    if (!fused) {  // the row's quantised query heads of this group, as the packing pass left them
        const size_t qrow = (size_t)(a.row0 + prow) * nh + (size_t)kvh * G;
        const int4* src = reinterpret_cast<const int4*>(a.q8 + qrow * HD);
        for (int i = tid; i < G * HD / 16; i += SPL_THREADS)
            reinterpret_cast<int4*>(&q8[0][0])[i] = src[i];
        if (tid < G) qsc[tid] = a.qsc[qrow + tid];
    }
    // heads past the group's real count: zero query (finite scores, never written out)
    for (int i = G * HD + tid; i < GT * HD; i += SPL_THREADS) (&q8[0][0])[i] = 0;
    if (tid < GT - G) qsc[G + tid] = 0.0f;
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
    float m_run[GT], l_run[GT], acc[GT][4];
#pragma unroll
    for (int g = 0; g < GT; g++) {
        m_run[g] = -__builtin_inff();
        l_run[g] = 0.0f;
        acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.0f;
    }
    // p.v mapping: thread = (dims 4*dg .. 4*dg+3, key subset ks)
    const int dg = tid % DG, ks = tid / DG;

    for (int t0 = j0; t0 < j1; t0 += SPL_THREADS) {
        const int j = t0 + tid;
        const bool live = j < j1;
        if (j == own) {
            ksj = kvs_new[0];
            vsj = kvs_new[1];
        }
        // 1. V pieces into the tile; each key's exact int32 q.k for every head of the group
#pragma unroll
        for (int u = 0; u < P; u++) {
            const int kt = u * KPR + kr;  // key in the tile
            if (t0 + kt == own) {
                kp[u] = *reinterpret_cast<const int4*>(knew + 16 * pc);
                vp[u] = *reinterpret_cast<const int4*>(vnew + 16 * pc);
            }
            *reinterpret_cast<int4*>(&vt[kt][16 * pc]) = vp[u];
            int dd[GT];
#pragma unroll
            for (int g = 0; g < GT; g++) {
                const int4 q4 = *reinterpret_cast<const int4*>(&q8[g][16 * pc]);
                int x = __builtin_amdgcn_sdot4(q4.x, kp[u].x, 0, false);
                x = __builtin_amdgcn_sdot4(q4.y, kp[u].y, x, false);
                x = __builtin_amdgcn_sdot4(q4.z, kp[u].z, x, false);
                x = __builtin_amdgcn_sdot4(q4.w, kp[u].w, x, false);
                dd[g] = piece_sum_last<P>(x);
            }
            if (pc == P - 1) {
                if constexpr (GT >= 4) {
#pragma unroll
                    for (int g = 0; g < GT; g += 4)
                        *reinterpret_cast<int4*>(&dots[kt][g]) = make_int4(dd[g], dd[g + 1], dd[g + 2], dd[g + 3]);
                } else {
#pragma unroll
                    for (int g = 0; g < GT; g++) dots[kt][g] = dd[g];
                }
            }
        }
        // the next tile's pieces and scales are independent of this one's math: request them now
        const int jn = j + SPL_THREADS;
        const bool next = jn < j1 && jn != own;
        if (t0 + SPL_THREADS < j1) load_tile(t0 + SPL_THREADS);
        const float ks_next = next ? KSc[jn] : 0.0f;
        const float vs_next = next ? VSc[jn] : 0.0f;
        __syncthreads();  // the tile's dots and V

        // 2. scores of this thread's key; tile maximum per head: waves, then the workgroup
        float sc[GT];
        {
            int dv[GT];
            if constexpr (GT >= 4) {
#pragma unroll
                for (int g = 0; g < GT; g += 4) {
                    const int4 t = *reinterpret_cast<const int4*>(&dots[tid][g]);
                    dv[g] = t.x;
                    dv[g + 1] = t.y;
                    dv[g + 2] = t.z;
                    dv[g + 3] = t.w;
                }
            } else {
#pragma unroll
                for (int g = 0; g < GT; g++) dv[g] = dots[tid][g];
            }
#pragma unroll
            for (int g = 0; g < GT; g++) sc[g] = live ? (float)dv[g] * ((ksj * qsc[g]) * scale) : -__builtin_inff();
        }
#pragma unroll
        for (int g = 0; g < GT; g++) {
            const float mw = wave_max64(sc[g]);
            if (lane == 0) redm[wave][g] = mw;
        }
        __syncthreads();
        // running maximum, the rescale of what came before, this tile's weights and sums
#pragma unroll
        for (int g = 0; g < GT; g++) {
            float mt = redm[0][g];
#pragma unroll
            for (int w = 1; w < NW; w++) mt = fmaxf(mt, redm[w][g]);
            const float mn = fmaxf(m_run[g], mt);
            const float al = m_run[g] == -__builtin_inff() ? 0.0f : exp_hw(m_run[g] - mn);
            m_run[g] = mn;
            const float e = live ? exp_hw(sc[g] - mn) : 0.0f;
            pw[g][tid] = e * vsj;
            l_run[g] *= al;
#pragma unroll
            for (int c = 0; c < 4; c++) acc[g][c] *= al;
            const float sw = wave_sum64(e);
            if (lane == 0) reds[wave][g] = sw;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < GT; g++) {
            float st = reds[0][g];
#pragma unroll
            for (int w = 1; w < NW; w++) st += reds[w][g];
            l_run[g] += st;
        }
        // 3. o[g][4dg + c] += sum over this subset's quads of keys of (e * vs) * v; the keys of
        // a quad past the tile's live ones carry zero weight
        const int tn = min(SPL_THREADS, j1 - t0);
        for (int q = ks; 4 * q < tn; q += NKS) {
            // the int8 values as v + 128 in unsigned bytes, converted and less 128 (exact).  The
            // direct (float)(int8) of a byte field compiled (hipcc 7.2, gfx950) to
            // v_cvt_f32_u32_sdwa with sext(), which converts a negative byte as 2^32 + v.
            unsigned v4[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v4[i] = *reinterpret_cast<const unsigned*>(&vt[4 * q + i][4 * dg]) ^ 0x80808080u;
            float4 p4[GT];
#pragma unroll
            for (int g = 0; g < GT; g++) p4[g] = *reinterpret_cast<const float4*>(&pw[g][4 * q]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float vv = (float)((v4[i] >> (8 * c)) & 0xffu) - 128.0f;
#pragma unroll
                    for (int g = 0; g < GT; g++) {
                        const float pg = i == 0 ? p4[g].x : i == 1 ? p4[g].y : i == 2 ? p4[g].z : p4[g].w;
                        acc[g][c] = __builtin_fmaf(pg, vv, acc[g][c]);
                    }
                }
            }
        }
        ksj = ks_next;
        vsj = vs_next;
        __syncthreads();  // the tile arrays are rewritten by the next tile or the subset sums
    }

    // the key subsets' sums, added in subset order
#pragma unroll
    for (int g = 0; g < GT; g++)
        *reinterpret_cast<float4*>(&accs[ks][g][4 * dg]) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
    __syncthreads();
    const int W = HD + 2;
    for (int o = tid; o < G * HD; o += SPL_THREADS) {
        const int g = o / HD, d = o - g * HD;
        float t = accs[0][g][d];
#pragma unroll
        for (int q = 1; q < NKS; q++) t += accs[q][g][d];
        if (!part) {  // the whole key range: the normalised output
            float lg = 0.0f;
#pragma unroll
            for (int gg = 0; gg < GT; gg++)
                if (gg == g) lg = l_run[gg];
            a.out[((size_t)(a.row0 + prow) * nh + kvh * G + g) * HD + d] = t / lg;
            continue;
        }
        float* out = part + ((size_t)(kvh * G + g) * ns + s) * W;
        act_st<COH>(out + d, t);
        if (d == 0) {
#pragma unroll
            for (int gg = 0; gg < GT; gg++)
                if (gg == g) {
                    act_st<COH>(out + HD, m_run[gg]);
                    act_st<COH>(out + HD + 1, l_run[gg]);
                }
        }
    }
    return true;
}

// Merge of the live slices of kv head kvh's G query heads into a.out, by one workgroup of
// SPL_THREADS threads (in the persistent decode kernel, the last slice workgroup of that kv
// head to finish): each slice's
// weight e^(m_s - M) and L = sum_s e^(m_s - M) l_s per head, then o = sum_s w_s o_s / L with
// SB slices' loads in flight per output.  LDS: ml [2 G live], wsl [G live] floats.  With
// COH the partials are read from the agent-coherent level (they were written by other
// workgroups) and the output written through to it.
template <int P, bool COH>
__device__ __forceinline__ void combine_group(const AttnArgs& a, int ns, const float* part, int kvh, float* ml,
                                              float* wsl) {
    constexpr int HD = P * 16;
    const int tid = threadIdx.x, G = a.nh / a.nkv, W = HD + 2;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + a.row0;
    const int nk = pos + 1;
    const int chunk = split_chunk(nk, ns);
    const int live = (nk + chunk - 1) / chunk;
    for (int i = tid; i < G * live; i += SPL_THREADS) {
        const int gg = i / live, s = i - gg * live;
        const float* o = part + ((size_t)(kvh * G + gg) * ns + s) * W;
        ml[2 * i] = act_ld<COH>(o + HD);
        ml[2 * i + 1] = act_ld<COH>(o + HD + 1);
    }
    __syncthreads();
    for (int i = tid; i < G * live; i += SPL_THREADS) {
        const int gg = i / live;
        float M = -__builtin_inff();
        for (int s = 0; s < live; s++) M = fmaxf(M, ml[2 * (gg * live + s)]);
        wsl[i] = exp_hw(ml[2 * i] - M);
    }
    __syncthreads();
    constexpr int SB = 16;
    for (int i = tid; i < G * HD; i += SPL_THREADS) {
        const int gg = i / HD, d = i - gg * HD;
        float L = 0.0f, o = 0.0f;
        const float* pb = part + (size_t)(kvh * G + gg) * ns * W;
        for (int s0 = 0; s0 < live; s0 += SB) {
            float ov[SB];
#pragma unroll
            for (int u = 0; u < SB; u++) ov[u] = s0 + u < live ? act_ld<COH>(pb + (size_t)(s0 + u) * W + d) : 0.0f;
#pragma unroll
            for (int u = 0; u < SB; u++)
                if (s0 + u < live) o = __builtin_fmaf(wsl[gg * live + s0 + u], ov[u], o);
        }
        for (int q = 0; q < live; q++) L = __builtin_fmaf(wsl[gg * live + q], ml[2 * (gg * live + q) + 1], L);
        act_st<COH>(a.out + (size_t)(kvh * G + gg) * HD + d, o / L);
    }
}

}  // namespace jy
