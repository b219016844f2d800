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
// Two kernels per layer (the matrix-core slice of jy_attention_mfma.h in both):
//  1. attn_split_kernel: one workgroup per (kv head, slice of keys).  It quantises the
//     group's query heads, walks its keys in 32-key steps per wave, and keeps a running
//     (max, sum, o[hd]) per query head of the group.  The workgroup whose slice holds the
//     token's own position appends its k and v to the cache and takes them from its own
//     copy, not from the cache row it is writing.
//  2. attn_combine_kernel: one workgroup per (query head, 32 dims) merges the slices:
//     M = max m_s, L = sum l_s e^(m_s - M), o = sum o_s e^(m_s - M) / L.
// Slices are a fixed count per launch (sized for the longest length a graph replay may
// see); the keys per slice follow the live length on the device, so a replayed step
// uses as many slices as that length needs.  Up to ATT_WHOLE_KEYS keys one kernel instead:
// attn_whole_kernel, one workgroup per (kv head, 16 output dims) over all the keys.
#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

#include "jy_attention_mfma.h"

namespace jy {

// P = hd / 16: 16-byte pieces per key row; GT = split_heads(query heads per kv head); NW
// waves per workgroup.  One workgroup per (kv head, slice); with one slice (part ==
// nullptr) the normalised output goes straight to a.out and no merge kernel follows.
// (Two forms whose last slice workgroup of each kv head merged the slices measured slower
// than the separate merge kernel: the partials' stores through the agent-coherent level,
// the count and the merge's coherent loads are three serial memory round trips.  8B decode
// after 1024 tokens: the VALU slice 386 vs 427 tokens/s; this slice 11.1 us vs 5.6 + 4.2.)
// waves per workgroup of the whole-range form (8 measured faster than 16 at 1024 keys, 10.3
// vs 12.0 us, and alike at 512)
static constexpr int WW = 8;

template <int P, int GT, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(4, 4))) void attn_split_kernel(
    AttnArgs a, int ns, float* __restrict__ part) {
    __shared__ MslLds<P * 16, NW> lds;
    attn_slice_mfma<P, GT, NW, false>(a, ns, part, blockIdx.x, blockIdx.y, lds);
}

// short ranges: one workgroup per (kv head, 16-dim tile of the output) over all the keys,
// WW waves, two steps of loads in flight per wave; no merge kernel
template <int P, int GT>
__global__ __launch_bounds__(64 * WW) __attribute__((amdgpu_waves_per_eu(4, 4))) void attn_whole_kernel(AttnArgs a) {
    __shared__ MslLds<P * 16, WW, 16> lds;
    attn_slice_mfma<P, GT, WW, false, P, 2>(a, 1, nullptr, blockIdx.x, 0, lds, 0, blockIdx.y);
}

// prompt rows: one workgroup per (kv head, R consecutive rows), the highest row's whole key
// range as one slice, the other rows' later keys masked per query column; the normalised
// output straight to a.out; row groups in descending order (the longest first).  R rows
// fill the 8 query columns of the slice's matrix operations (R x the group's heads).
template <int P, int R>
__global__ __launch_bounds__(SPL_THREADS) __attribute__((amdgpu_waves_per_eu(4, 4))) void attn_prefill_kernel(AttnArgs a) {
    __shared__ MslLds<P * 16, 4> lds;
    attn_slice_mfma<P, SPL_GMAX, 4, false, 1, 1, R>(a, 1, nullptr, blockIdx.x, 0, lds,
                                                    a.nrows - 1 - R * (int)blockIdx.y);
}

// The merge for many slices: one workgroup per (query head, 32 output dims).  Every load
// goes out first (thread (d, group q) holds o_s[d] of slices q, q+8, ..., q+248 in
// registers, thread t the (max, sum) of slice t), so the merge costs one memory round trip;
// then M and L from all live slices' (max, sum) and the weighted sum, the 8 groups added in
// order.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a, int ns, const float* __restrict__ part) {
    __shared__ float wsl[256], red[8][32], redl[4], redm[4];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hd = a.hd, W = hd + 2;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + a.row0;
    const int nk = pos + 1;
    const int chunk = split_chunk(nk, ns);
    const int live = (nk + chunk - 1) / chunk;  // <= ns <= 256
    const float* p = part + (size_t)h * ns * W;
    const int d = blockIdx.y * 32 + (tid & 31), q = tid >> 5;
    float ov[32];
#pragma unroll
    for (int k = 0; k < 32; k++) ov[k] = q + 8 * k < live ? p[(size_t)(q + 8 * k) * W + d] : 0.0f;
    const float ms = tid < live ? p[(size_t)tid * W + hd] : -__builtin_inff();
    const float ls = tid < live ? p[(size_t)tid * W + hd + 1] : 0.0f;
    const float mw = wave_max64(ms);
    if (lane == 0) redm[wave] = mw;
    __syncthreads();
    const float M = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    const float w = tid < live ? exp_hw(ms - M) : 0.0f;
    wsl[tid] = w;
    const float lw = wave_sum64(w * ls);
    if (lane == 0) redl[wave] = lw;
    __syncthreads();
    const float L = (redl[0] + redl[1]) + (redl[2] + redl[3]);
    float o = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) o = __builtin_fmaf(wsl[(q + 8 * k) & 255], ov[k], o);  // (0 past live)
    red[q][tid & 31] = o;
    __syncthreads();
    if (tid < 32) {
        float t = red[0][tid];
#pragma unroll
        for (int k = 1; k < 8; k++) t += red[k][tid];
        a.out[(size_t)h * hd + d] = t / L;
    }
}

bool attn_split_supported(int nh, int nkv, int hd) {
    return nkv > 0 && nh % nkv == 0 && nh / nkv <= SPL_GMAX && (hd == 64 || hd == 128);
}

// Slices: one 32-key step per wave.  Up to MSL_WIDE_KEYS keys (the most a launch may see),
// workgroups of 4 waves over 128-key slices; beyond, 8 waves over 256-key slices (half the
// slices for the merge to read: Qwen2.5-7B decode after 32768 positions 409 -> 418 tokens/s;
// at Llama-3-8B's 1024 keys the 4-wave form is faster, 438 vs 434).  A second step of a
// wave waits a whole memory round trip, which measured slower than more workgroups and the
// merge kernel (16 waves x 64 keys per kv head at 1024 keys 14.1 us vs 7.0 + 4.6 us).
static constexpr int MSL_WIDE_KEYS = 8192;

static int slice_keys(int max_keys) { return max_keys > MSL_WIDE_KEYS ? 256 : 128; }

int attn_split_slices(int keys) {
    const int sk = slice_keys(keys);
    return std::max(1, std::min(256, (keys + sk - 1) / sk));
}

size_t attn_split_part_floats(int nh, int hd, int ns) { return (size_t)nh * ns * (hd + 2); }

// Workgroups of kernel k that the device holds at once (occupancy per CU times the CUs),
// asked once per kernel.  The slice count is capped at that over the kv heads: a grid one
// workgroup past it waits for a whole workgroup's time at the end (Qwen2.5-7B at 32769..32895
// keys: 4 kv heads x 129 slices of 256 keys = 516 workgroups for 512 places).
template <typename K>
static int resident_wgs(K k, int threads) {
    static std::mutex mu;
    static std::vector<std::pair<const void*, int>> known;
    std::lock_guard<std::mutex> g(mu);
    for (const auto& e : known)
        if (e.first == (const void*)k) return e.second;
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, threads, 0) != hipSuccess || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 1 << 30;  // (no cap: the launch itself reports the device's error)
    const int n = std::max(1, per_cu) * cus;
    known.emplace_back((const void*)k, n);
    return n;
}

template <int NW>
static int split_launch(const AttnArgs& a, float* part, int ns, hipStream_t st) {
    auto k = attn_split_kernel<8, 8, NW>;
    switch (split_heads(a.nh / a.nkv) * (a.hd == 64 ? -1 : 1)) {
        case -1: k = attn_split_kernel<4, 1, NW>; break;
        case -2: k = attn_split_kernel<4, 2, NW>; break;
        case -4: k = attn_split_kernel<4, 4, NW>; break;
        case -8: k = attn_split_kernel<4, 8, NW>; break;
        case 1: k = attn_split_kernel<8, 1, NW>; break;
        case 2: k = attn_split_kernel<8, 2, NW>; break;
        case 4: k = attn_split_kernel<8, 4, NW>; break;
        default: break;
    }
    ns = std::max(1, std::min(ns, resident_wgs(k, 64 * NW) / a.nkv));
    hipLaunchKernelGGL(k, dim3(a.nkv, ns), dim3(64 * NW), 0, st, a, ns, ns > 1 ? part : nullptr);
    return ns;
}

// the slices (the form by a.max_keys, the longest length the launch may see; at most ns, and
// no more than the device holds at once), then (more than one) the merge over (head, 32 dims)
void launch_attention_split(const AttnArgs& a, float* part, int ns, hipStream_t st) {
    ns = slice_keys(a.max_keys) > 128 ? split_launch<8>(a, part, ns, st) : split_launch<4>(a, part, ns, st);
    if (ns > 1) hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nh, a.hd / 32), dim3(256), 0, st, a, ns, part);
}

// Up to this many keys a decode row takes the whole-range form (one launch, 64 workgroups at
// Llama-3-8B's shape), beyond it the slices and the merge.  Every workgroup of a kv head
// runs the q.k and softmax of all its keys, so the form's time grows with the keys about
// twice as fast as the split form's (Llama-3-8B shape: 6.7 us at 512 keys, 10.3 at 1024,
// 13.7 at 2048 vs 5.9 + 4.7 for the slices and merge at 1024); Qwen2.5-0.5B decode
// after 512 positions 1340 -> 1405 tokens/s.
static constexpr int ATT_WHOLE_KEYS = 1024;

int att_whole_keys() { return ATT_WHOLE_KEYS; }

void launch_attention_whole(const AttnArgs& a, hipStream_t st) {
    auto k = attn_whole_kernel<8, 8>;
    switch (split_heads(a.nh / a.nkv) * (a.hd == 64 ? -1 : 1)) {
        case -1: k = attn_whole_kernel<4, 1>; break;
        case -2: k = attn_whole_kernel<4, 2>; break;
        case -4: k = attn_whole_kernel<4, 4>; break;
        case -8: k = attn_whole_kernel<4, 8>; break;
        case 1: k = attn_whole_kernel<8, 1>; break;
        case 2: k = attn_whole_kernel<8, 2>; break;
        case 4: k = attn_whole_kernel<8, 4>; break;
        default: break;
    }
    hipLaunchKernelGGL(k, dim3(a.nkv, a.hd / 16), dim3(64 * WW), 0, st, a);
}

// Rows per workgroup: as many as the 8 query columns hold (R = 8 / split_heads(G)).
// Llama-3-8B shape (4 query heads per kv head), 1024 prompt rows: one row per workgroup
// 108 us per layer, two rows [measured below].
void launch_attention_prefill_split(const AttnArgs& a, hipStream_t st) {
    const int R = SPL_GMAX / split_heads(a.nh / a.nkv);
    const dim3 grid(a.nkv, (a.nrows + R - 1) / R), block(SPL_THREADS);
    auto k = attn_prefill_kernel<8, 1>;
    switch (R * (a.hd == 64 ? -1 : 1)) {
        case -1: k = attn_prefill_kernel<4, 1>; break;
        case -2: k = attn_prefill_kernel<4, 2>; break;
        case -4: k = attn_prefill_kernel<4, 4>; break;
        case -8: k = attn_prefill_kernel<4, 8>; break;
        case 2: k = attn_prefill_kernel<8, 2>; break;
        case 4: k = attn_prefill_kernel<8, 4>; break;
        case 8: k = attn_prefill_kernel<8, 8>; break;
        default: break;
    }
    hipLaunchKernelGGL(k, grid, block, 0, st, a);
}

}  // namespace jy
