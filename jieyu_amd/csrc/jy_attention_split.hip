// jy_attention_split.hip — decode attention over the int8 KV cache split across
// workgroups (flash-decoding): the tolerance mode's form of attention_q8
// (libs/model_libs/attention/attention_q8.h:38-184, attention/x86/x86_classic.txt:14-73).
//
// What it keeps from the reference: q, and the token's k and v, quantised to int8
// per head (absmax / 127, lrintf, kv_pack_q8 at attention_q8.h:20-37); the exact int32
// q.k dot; score = (float)dot * ((ks * qsc) * (1/sqrtf(hd))); e = expf(score - max)
// with glibc's expf.  What it reorders: the softmax sum and the p.v accumulation run
// per slice of keys and are merged afterwards, so their fp32 rounding differs from the
// reference's single ascending chains (a few ulp of the result).
//
// Two kernels per layer.
//  1. attn_split_kernel: one workgroup per (kv head, slice of keys).  It quantises the
//     group's query heads, walks its keys in tiles of one key per thread (K and V rows
//     straight into registers), and keeps a running (max, sum, o[hd]) per query head
//     of the group, rescaled per tile.  The workgroup whose slice holds the token's own
//     position quantises its k and v, appends them to the cache and uses its own copy.
//  2. attn_combine_kernel: one workgroup per query head merges the slices:
//     M = max m_s, L = sum l_s e^(m_s - M), o = sum o_s e^(m_s - M) / L.
// Slices are a fixed count per launch (sized for the longest length a graph replay may
// see); the keys per slice follow the live length on the device, so a replayed step
// uses as many slices as that length needs.
#include <algorithm>

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

// P = hd / 16: 16-byte pieces per key row
template <int P>
__global__ __launch_bounds__(SPL_THREADS) void attn_split_kernel(AttnArgs a, int ns, float* __restrict__ part) {
    constexpr int HD = P * 16;
    constexpr int NW = SPL_THREADS / 64;
    constexpr int KS = SPL_THREADS / HD;  // key subsets of the p.v phase (4 for hd 64, 2 for hd 128)
    __shared__ __align__(16) int8_t q8[SPL_GMAX][HD];
    __shared__ float qsc[SPL_GMAX];
    __shared__ __align__(16) int8_t vt[SPL_THREADS][HD + 16];  // V tile, rows padded
    __shared__ float pw[SPL_GMAX][SPL_THREADS];                 // e_j * vs_j of the tile
    __shared__ float redm[NW][SPL_GMAX], reds[NW][SPL_GMAX];
    __shared__ __align__(16) int8_t knew[HD], vnew[HD];
    __shared__ float kvs_new[2];
    __shared__ float accs[KS - 1][SPL_GMAX][HD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nh = a.nh, nkv = a.nkv, G = nh / nkv;
    const int kvh = blockIdx.x, s = blockIdx.y;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + a.row0;
    const int nk = pos + 1;
    const int chunk = split_chunk(nk, ns);
    const int j0 = s * chunk;
    if (j0 >= nk) return;  // whole workgroup: a slice past the live length
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
            for (int c = 0; c < PER; c++) qv[t][c] = src[lane + 64 * c];
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
                o[d] = acc[g];
                if (d == 0) {
                    o[HD] = m_run[g];
                    o[HD + 1] = l_run[g];
                }
            }
    }
}

// one workgroup of 256 threads per query head merges the live slices: every slice's
// (max, sum) loaded at once, the weights e^(m_s - M) one per thread, then o over the
// slices in two interleaved halves per output dim, summed in a fixed order
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a, int ns, const float* __restrict__ part) {
    __shared__ float wsl[256], lsl[256], red[4];
    __shared__ float half_o[256];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hd = a.hd, W = hd + 2;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + a.row0;
    const int nk = pos + 1;
    const int chunk = split_chunk(nk, ns);
    const int live = (nk + chunk - 1) / chunk;  // <= ns <= 256
    const float* p = part + (size_t)h * ns * W;
    const float ms = tid < live ? p[(size_t)tid * W + hd] : -__builtin_inff();
    const float ls = tid < live ? p[(size_t)tid * W + hd + 1] : 0.0f;
    const float mw = wave_max64(ms);
    if (lane == 0) red[wave] = mw;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float w = tid < live ? exp_hw(ms - M) : 0.0f;
    wsl[tid] = w;
    lsl[tid] = w * ls;
    __syncthreads();
    // L: fixed-order sum of w_s * l_s
    float L = 0.0f;
    for (int s = 0; s < live; s++) L += lsl[s];
    // thread (d, half): slices half, half + 2, ... with four loads in flight
    const int nd = hd, dd = tid % nd, hf = tid / nd;  // hd 64: four quarters; hd 128: two halves
    const int nsub = 256 / nd;
    float o = 0.0f;
    int s = hf;
    for (; s + 3 * nsub < live; s += 4 * nsub) {
        const float o0 = p[(size_t)s * W + dd], o1 = p[(size_t)(s + nsub) * W + dd];
        const float o2 = p[(size_t)(s + 2 * nsub) * W + dd], o3 = p[(size_t)(s + 3 * nsub) * W + dd];
        o = __builtin_fmaf(wsl[s], o0, o);
        o = __builtin_fmaf(wsl[s + nsub], o1, o);
        o = __builtin_fmaf(wsl[s + 2 * nsub], o2, o);
        o = __builtin_fmaf(wsl[s + 3 * nsub], o3, o);
    }
    for (; s < live; s += nsub) o = __builtin_fmaf(wsl[s], p[(size_t)s * W + dd], o);
    half_o[tid] = o;
    __syncthreads();
    if (tid < nd) {
        float t = half_o[tid];
        for (int q = 1; q < nsub; q++) t += half_o[q * nd + tid];
        a.out[(size_t)h * hd + tid] = t / L;
    }
}

bool attn_split_supported(int nh, int nkv, int hd) {
    return nkv > 0 && nh % nkv == 0 && nh / nkv <= SPL_GMAX && (hd == 64 || hd == 128);
}

int attn_split_slices(int keys) { return std::max(1, std::min(256, (keys + 127) / 128)); }

size_t attn_split_part_floats(int nh, int hd, int ns) { return (size_t)nh * ns * (hd + 2); }

void launch_attention_split(const AttnArgs& a, float* part, int ns, hipStream_t st) {
    const dim3 grid(a.nkv, ns), block(SPL_THREADS);
    if (a.hd == 64)
        hipLaunchKernelGGL(attn_split_kernel<4>, grid, block, 0, st, a, ns, part);
    else
        hipLaunchKernelGGL(attn_split_kernel<8>, grid, block, 0, st, a, ns, part);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nh), dim3(256), 0, st, a, ns, part);
}

}  // namespace jy
