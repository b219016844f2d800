// jy_attention.hip — GQA attention over the int8 KV cache, bit-exact with
// attention_q8 (libs/model_libs/attention/attention_q8.h:20-37, :38-184 and
// attention/x86/x86_classic.txt:10-73):
//   Q -> int8 per head (absmax, lrintf); exact int32 q.k for every key j <= p;
//   score_j = (float)dot * ((ks_j * qsc) * (1/sqrtf(hd))); strict max from -1e30;
//   e_j = expf(score_j - max); sum += e_j in ascending j; p_j = e_j * (1/sum);
//   o[d] = fma(p_j * vs_j, (float)v8[j][d], o[d]) in ascending j.
//
// Two kernels per attention call.
//  1. attn_scores_kernel: one workgroup per (kv head, run of keys, token row)
//     computes the scores of every query head of the GQA group against its keys,
//     so each key is read once per group.  A key's bytes are spread over adjacent
//     lanes (16 B each: 8 lanes per 128-byte key), the loads are coalesced and the
//     lanes combine their partial int32 dots with butterflies.  In the fused decode
//     form it also quantises the token's q, k and v, and one workgroup per kv head
//     appends k/v to the cache (kv_pack_q8 of the new position).
//  2. attn_softmax_pv_kernel: one workgroup per (query head, token row, slice of
//     output dims) runs the reference's two ascending chains on wave 0: the softmax
//     sum on one lane, then one lane per output dim, while waves 1..7 stage this
//     slice of V in LDS (fp16, exact for int8, rows padded so the chain's 16-byte
//     reads do not collide in a bank).  Up to ATT_ECAP keys every e_j stays in LDS;
//     past it e_j, p_j * vs_j and V move through double-buffered windows, so the
//     chains run back to back while the other waves fill the next buffer.
// Scores travel between the two through a per-row [nh][max_keys] float array.
// A decode token attending at most ATT_ONE keys takes one kernel instead:
// attn_softmax_pv_kernel<true> computes its head's scores itself (att_scores_local),
// with the first workgroup of each kv head appending the new K/V slot.
#include "jy_layout.h"

namespace jy {

static constexpr int ATT_THREADS = 256;
static constexpr int SPV_THREADS = 512;  // softmax/PV: wave 0 runs a chain, waves 1..7 feed it
static constexpr int ATT_ECAP = 1536;  // keys kept in LDS whole; past this the windowed form (faster there)
// decode steps up to this many keys compute the scores inside the softmax/PV workgroups
// (one kernel); past it every workgroup re-reading its kv head's whole key run costs
// more than the second launch (measured: one kernel 12.4 vs 14.8 us at 512 keys, 18.4
// vs 18.0 at 1024)
static constexpr int ATT_ONE = 768;
static constexpr int ATT_LW = 1536;    // sum-chain window past that
static constexpr int ATT_LC = 1024;    // largest PV chunk past that
constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
static constexpr int ATT_GB = 8;       // query heads per scores workgroup
static constexpr int ATT_U = 2;        // key loads per lane in the scores kernel

// ------------------------------------------------------------------ scores

// Sum of each group of LP adjacent lanes (LP a power of two, at most 16) into the
// group's last lane, by DPP row shifts (exact: integer adds).
__device__ __forceinline__ int group_sum_last(int d, int LP) {
    if (LP > 1) d += __builtin_amdgcn_update_dpp(0, d, 0x111, 0xf, 0xf, true);  // row_shr:1
    if (LP > 2) d += __builtin_amdgcn_update_dpp(0, d, 0x112, 0xf, 0xf, true);  // row_shr:2
    if (LP > 4) d += __builtin_amdgcn_update_dpp(0, d, 0x114, 0xf, 0xf, true);  // row_shr:4
    if (LP > 8) d += __builtin_amdgcn_update_dpp(0, d, 0x118, 0xf, 0xf, true);  // row_shr:8
    return d;
}


__global__ __launch_bounds__(ATT_THREADS) void attn_scores_kernel(AttnArgs a, int kc) {
    __shared__ __align__(16) int8_t qv8[ATT_GB][256];
    __shared__ __align__(16) int8_t kloc[256];
    __shared__ __align__(16) int8_t vloc[256];
    __shared__ float qsc[ATT_GB];
    __shared__ float kvsc[2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int hd = a.hd, nh = a.nh, nkv = a.nkv, group = nh / nkv;
    const int nb = (group + ATT_GB - 1) / ATT_GB;
    const int kvh = blockIdx.x / nb, hb = blockIdx.x - kvh * nb;
    const int h0 = kvh * group + hb * ATT_GB;
    const int gh = min(ATT_GB, group - hb * ATT_GB);
    const int rr = blockIdx.z, r = a.row0 + rr;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + r;
    const int nk = pos + 1;
    const int j0 = blockIdx.y * kc;
    const bool fused = a.fused;
    const bool appender = fused && blockIdx.y == 0 && hb == 0;
    if (j0 >= nk) return;  // whole workgroup: no key of this run is attended (run 0 always is)
    const int jend = min(j0 + kc, nk);
    const size_t head = (size_t)a.layer * nkv + kvh;
    const int8_t* K = a.kv.k + head * a.kv.max_seq * hd;
    const float* KS = a.kv.ks + head * a.kv.max_seq;

    // ---- the keys first: their loads depend only on the position, so they are in
    // flight while the token's vectors are quantised.  One key's 16-byte pieces sit
    // on LP adjacent lanes (the pieces of hd rounded up to a power of two); a wave
    // covers KW = 64/LP keys per load and each lane ATT_U loads (kc = 4*KW*ATT_U).
    const bool vec = (hd & 15) == 0;
    const int P = hd >> 4;
    int LP = 1;
    while (LP < P) LP <<= 1;
    const int KW = 64 / LP, piece = lane & (LP - 1), kl = lane / LP;
    const bool live = vec && piece < P;
    int4 k4[ATT_U];
    float ksv[ATT_U];
#pragma unroll
    for (int u = 0; u < ATT_U; u++) {
        const int j = j0 + (u * (ATT_THREADS / 64) + wave) * KW + kl;
        const int jc = min(j, jend - 1);
        k4[u] = live ? *reinterpret_cast<const int4*>(K + (size_t)jc * hd + piece * 16) : make_int4(0, 0, 0, 0);
        ksv[u] = vec ? KS[jc] : 0.0f;
    }

    // ---- this token's q (and, fused, k and v) as int8: absmax, lrintf (kv_pack_q8,
    // attention_q8.h:29-35); wave w takes items w, w+4, w+8 with all their loads
    // issued before the reductions
    if (fused) {
        const float* row = a.qkv + (size_t)rr * (nh + 2 * nkv) * hd;
        const int nitems = gh + 2;  // query heads, then k, then v
        float vals[3][4];
#pragma unroll
        for (int t = 0; t < 3; t++) {
            const int i = wave + 4 * t;
            if (i < nitems) {
                const float* src = i < gh ? row + (size_t)(h0 + i) * hd
                                          : row + (size_t)((i == gh ? nh : nh + nkv) + kvh) * hd;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int d = lane + 64 * c;
                    vals[t][c] = d < hd ? src[d] : 0.0f;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 3; t++) {
            const int i = wave + 4 * t;
            if (i < nitems) {
                float amax = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; c++) amax = fmaxf(amax, fabsf(vals[t][c]));
                amax = wave_max64(amax);
                const float inv = quant_inv(amax);
                int8_t* dst = i < gh ? qv8[i] : (i == gh ? kloc : vloc);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int d = lane + 64 * c;
                    if (d < hd) dst[d] = quant_i8(vals[t][c], inv);
                }
                if (lane == 0) {
                    if (i < gh)
                        qsc[i] = quant_scale(amax);
                    else
                        kvsc[i - gh] = quant_scale(amax);
                }
            }
        }
    } else {
        for (int i = tid; i < gh * hd; i += blockDim.x) {
            const int hh = i / hd, d = i - hh * hd;
            qv8[hh][d] = a.q8[((size_t)r * nh + h0 + hh) * hd + d];
        }
        if (tid < gh) qsc[tid] = a.qsc[(size_t)r * nh + h0 + tid];
    }
    __syncthreads();
    if (appender) {  // kv_pack_q8 of the new position, once per kv head
        const size_t slot = head * a.kv.max_seq + pos;
        for (int d = tid; d < hd; d += blockDim.x) {
            a.kv.k[slot * hd + d] = kloc[d];
            a.kv.v[slot * hd + d] = vloc[d];
        }
        if (tid == 0) {
            a.kv.ks[slot] = kvsc[0];
            a.kv.vs[slot] = kvsc[1];
        }
    }

    float* S = a.scratch + ((size_t)rr * nh + h0) * a.max_keys;
    const float scale = 1.0f / sqrtf((float)hd);
    if (vec) {
        int4 qw[ATT_GB];  // this lane's piece of every query head (pieces < P only: no read past hd)
#pragma unroll
        for (int hh = 0; hh < ATT_GB; hh++)
            qw[hh] = (live && hh < gh) ? *reinterpret_cast<const int4*>(&qv8[hh][piece * 16]) : make_int4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < ATT_U; u++) {
            const int j = j0 + (u * (ATT_THREADS / 64) + wave) * KW + kl;
            if (fused && j == pos) {  // the new key is not in the cache yet
                k4[u] = live ? *reinterpret_cast<const int4*>(&kloc[piece * 16]) : make_int4(0, 0, 0, 0);
                ksv[u] = kvsc[0];
            }
            int dot[ATT_GB];
#pragma unroll
            for (int hh = 0; hh < ATT_GB; hh++) {
                int d = __builtin_amdgcn_sdot4(qw[hh].x, k4[u].x, 0, false);
                d = __builtin_amdgcn_sdot4(qw[hh].y, k4[u].y, d, false);
                d = __builtin_amdgcn_sdot4(qw[hh].z, k4[u].z, d, false);
                d = __builtin_amdgcn_sdot4(qw[hh].w, k4[u].w, d, false);
                dot[hh] = group_sum_last(d, LP);
            }
            if (piece == LP - 1 && j < jend) {
#pragma unroll
                for (int hh = 0; hh < ATT_GB; hh++)
                    if (hh < gh) S[(size_t)hh * a.max_keys + j] = (float)dot[hh] * ((ksv[u] * qsc[hh]) * scale);
            }
        }
    } else {
        // head dims that are not a multiple of 16: one lane per key, 4-byte words
        for (int j = j0 + tid; j < jend; j += blockDim.x) {
            const bool here = fused && j == pos;
            const int32_t* k32 = here ? reinterpret_cast<const int32_t*>(kloc)
                                      : reinterpret_cast<const int32_t*>(K + (size_t)j * hd);
            const float ksj = here ? kvsc[0] : KS[j];
            for (int hh = 0; hh < gh; hh++) {
                const int32_t* q32 = reinterpret_cast<const int32_t*>(qv8[hh]);
                int dot = 0;
                for (int i = 0; i < (hd >> 2); i++) dot = __builtin_amdgcn_sdot4(q32[i], k32[i], dot, false);
                S[(size_t)hh * a.max_keys + j] = (float)dot * ((ksj * qsc[hh]) * scale);
            }
        }
    }
}

// ------------------------------------------------------------------ softmax + PV

// byte address of an LDS object for ds_* instructions (the local-address-space view
// of a generic pointer into __shared__ memory)
__device__ __forceinline__ uint32_t lds_off(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// The two sequential chains of the reference softmax/PV, one dependent VALU op per
// step, written as GCN assembly: the compiler turns a C ping-pong of register
// arrays into one register copy per step.  The loops are short and fixed, and wait
// on lgkmcnt only for the register set they are about to read (LDS returns in
// order); the tails are C.
//
// sum += e[j], j ascending (libs/model_libs/attention/x86/x86_classic.txt:55-58).
// Lanes 0..15 of the calling wave read 64 consecutive e values with one
// ds_read_b128 (lane k holds e[4k .. 4k+3]) and lane 0 adds them in order, taking
// lane k's registers with a DPP row shift: one LDS read per 64 steps.  Two 64-step
// register sets, one in flight while the other is consumed (the last set may be
// read past n, inside the caller's LDS allocation, and is then unused).  Lanes
// 1..15 compute values that are discarded; lane 0 returns the sum.
__device__ __forceinline__ float chain_sum16(const float* e, int n, float sum) {
    int nb = n >> 6;
    if (nb > 0) {
        uint32_t pa = lds_off(e) + 16u * (threadIdx.x & 15u);
        asm volatile(
        "s_waitcnt lgkmcnt(0)\n"
        "ds_read_b128 v[100:103], %[pa]\n"
        "ds_read_b128 v[104:107], %[pa] offset:256\n"
        "s_sub_u32 %[nb], %[nb], 1\n"
        "L_s16_loop_%=:\n"
        "s_cmp_eq_u32 %[nb], 0\n"
        "s_cbranch_scc1 L_s16_lastA_%=\n"
        "s_waitcnt lgkmcnt(1)\n"
        "v_add_f32 %[s], v100, %[s]\n"
        "v_add_f32 %[s], v101, %[s]\n"
        "v_add_f32 %[s], v102, %[s]\n"
        "v_add_f32 %[s], v103, %[s]\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_u32_e32 %[pa], 0x200, %[pa]\n"
        "ds_read_b128 v[100:103], %[pa]\n"
        "s_sub_u32 %[nb], %[nb], 1\n"
        "s_cmp_eq_u32 %[nb], 0\n"
        "s_cbranch_scc1 L_s16_lastB_%=\n"
        "s_waitcnt lgkmcnt(1)\n"
        "v_add_f32 %[s], v104, %[s]\n"
        "v_add_f32 %[s], v105, %[s]\n"
        "v_add_f32 %[s], v106, %[s]\n"
        "v_add_f32 %[s], v107, %[s]\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "ds_read_b128 v[104:107], %[pa] offset:256\n"
        "s_sub_u32 %[nb], %[nb], 1\n"
        "s_branch L_s16_loop_%=\n"
        "L_s16_lastB_%=:\n"
        "s_waitcnt lgkmcnt(0)\n"
        "v_add_f32 %[s], v104, %[s]\n"
        "v_add_f32 %[s], v105, %[s]\n"
        "v_add_f32 %[s], v106, %[s]\n"
        "v_add_f32 %[s], v107, %[s]\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v104, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v105, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v106, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v107, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "s_branch L_s16_end_%=\n"
        "L_s16_lastA_%=:\n"
        "s_waitcnt lgkmcnt(0)\n"
        "v_add_f32 %[s], v100, %[s]\n"
        "v_add_f32 %[s], v101, %[s]\n"
        "v_add_f32 %[s], v102, %[s]\n"
        "v_add_f32 %[s], v103, %[s]\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:1 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:2 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:3 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:4 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:5 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:6 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:7 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:8 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:9 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:10 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:11 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:12 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:13 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:14 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v100, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v101, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v102, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "v_add_f32_dpp %[s], v103, %[s] row_shl:15 row_mask:0xf bank_mask:0xf\n"
        "L_s16_end_%=:\n"
        : [s] "+v"(sum), [pa] "+v"(pa), [nb] "+s"(nb)
        :
        : "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "scc", "memory");
    }
    for (int j = n & ~63; j < n; j++) sum += e[j];
    return sum;
}

// o = fma(p_j, v_j, o), j ascending; v as fp16 (exact for int8), so each step is one
// v_fma_mix (libs/model_libs/attention/x86/x86_classic.txt:63-70).  Operands stream
// through two register sets of 32 steps.
__device__ __forceinline__ float chain_pv(const float* P, const _Float16* vr, float o, int n) {
    int nb = n >> 6;
    if (nb > 0) {
        uint32_t pa = lds_off(P), va = lds_off(vr);
        asm volatile(
        "s_waitcnt lgkmcnt(0)\n"
        "ds_read_b128 v[100:103], %[pa]\n"
        "ds_read_b128 v[104:107], %[pa] offset:16\n"
        "ds_read_b128 v[108:111], %[pa] offset:32\n"
        "ds_read_b128 v[112:115], %[pa] offset:48\n"
        "ds_read_b128 v[116:119], %[pa] offset:64\n"
        "ds_read_b128 v[120:123], %[pa] offset:80\n"
        "ds_read_b128 v[124:127], %[pa] offset:96\n"
        "ds_read_b128 v[128:131], %[pa] offset:112\n"
        "ds_read_b128 v[132:135], %[va]\n"
        "ds_read_b128 v[136:139], %[va] offset:16\n"
        "ds_read_b128 v[140:143], %[va] offset:32\n"
        "ds_read_b128 v[144:147], %[va] offset:48\n"
        "ds_read_b128 v[148:151], %[pa] offset:128\n"
        "ds_read_b128 v[152:155], %[pa] offset:144\n"
        "ds_read_b128 v[156:159], %[pa] offset:160\n"
        "ds_read_b128 v[160:163], %[pa] offset:176\n"
        "ds_read_b128 v[164:167], %[pa] offset:192\n"
        "ds_read_b128 v[168:171], %[pa] offset:208\n"
        "ds_read_b128 v[172:175], %[pa] offset:224\n"
        "ds_read_b128 v[176:179], %[pa] offset:240\n"
        "ds_read_b128 v[180:183], %[va] offset:64\n"
        "ds_read_b128 v[184:187], %[va] offset:80\n"
        "ds_read_b128 v[188:191], %[va] offset:96\n"
        "ds_read_b128 v[192:195], %[va] offset:112\n"
        "s_sub_u32 %[nb], %[nb], 1\n"
        "L_pv_loop_%=:\n"
        "s_cmp_eq_u32 %[nb], 0\n"
        "s_cbranch_scc1 L_pv_last_%=\n"
        "s_waitcnt lgkmcnt(12)\n"
        "v_fma_mix_f32 %[o], v100, v132, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v101, v132, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v102, v133, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v103, v133, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v104, v134, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v105, v134, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v106, v135, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v107, v135, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v108, v136, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v109, v136, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v110, v137, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v111, v137, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v112, v138, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v113, v138, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v114, v139, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v115, v139, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v116, v140, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v117, v140, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v118, v141, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v119, v141, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v120, v142, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v121, v142, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v122, v143, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v123, v143, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v124, v144, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v125, v144, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v126, v145, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v127, v145, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v128, v146, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v129, v146, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v130, v147, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v131, v147, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_add_u32_e32 %[pa], 0x100, %[pa]\n"
        "v_add_u32_e32 %[va], 0x80, %[va]\n"
        "ds_read_b128 v[100:103], %[pa]\n"
        "ds_read_b128 v[104:107], %[pa] offset:16\n"
        "ds_read_b128 v[108:111], %[pa] offset:32\n"
        "ds_read_b128 v[112:115], %[pa] offset:48\n"
        "ds_read_b128 v[116:119], %[pa] offset:64\n"
        "ds_read_b128 v[120:123], %[pa] offset:80\n"
        "ds_read_b128 v[124:127], %[pa] offset:96\n"
        "ds_read_b128 v[128:131], %[pa] offset:112\n"
        "ds_read_b128 v[132:135], %[va]\n"
        "ds_read_b128 v[136:139], %[va] offset:16\n"
        "ds_read_b128 v[140:143], %[va] offset:32\n"
        "ds_read_b128 v[144:147], %[va] offset:48\n"
        "s_waitcnt lgkmcnt(12)\n"
        "v_fma_mix_f32 %[o], v148, v180, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v149, v180, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v150, v181, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v151, v181, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v152, v182, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v153, v182, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v154, v183, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v155, v183, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v156, v184, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v157, v184, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v158, v185, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v159, v185, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v160, v186, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v161, v186, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v162, v187, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v163, v187, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v164, v188, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v165, v188, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v166, v189, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v167, v189, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v168, v190, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v169, v190, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v170, v191, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v171, v191, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v172, v192, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v173, v192, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v174, v193, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v175, v193, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v176, v194, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v177, v194, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v178, v195, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v179, v195, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "ds_read_b128 v[148:151], %[pa] offset:128\n"
        "ds_read_b128 v[152:155], %[pa] offset:144\n"
        "ds_read_b128 v[156:159], %[pa] offset:160\n"
        "ds_read_b128 v[160:163], %[pa] offset:176\n"
        "ds_read_b128 v[164:167], %[pa] offset:192\n"
        "ds_read_b128 v[168:171], %[pa] offset:208\n"
        "ds_read_b128 v[172:175], %[pa] offset:224\n"
        "ds_read_b128 v[176:179], %[pa] offset:240\n"
        "ds_read_b128 v[180:183], %[va] offset:64\n"
        "ds_read_b128 v[184:187], %[va] offset:80\n"
        "ds_read_b128 v[188:191], %[va] offset:96\n"
        "ds_read_b128 v[192:195], %[va] offset:112\n"
        "s_sub_u32 %[nb], %[nb], 1\n"
        "s_branch L_pv_loop_%=\n"
        "L_pv_last_%=:\n"
        "s_waitcnt lgkmcnt(12)\n"
        "v_fma_mix_f32 %[o], v100, v132, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v101, v132, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v102, v133, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v103, v133, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v104, v134, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v105, v134, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v106, v135, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v107, v135, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v108, v136, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v109, v136, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v110, v137, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v111, v137, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v112, v138, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v113, v138, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v114, v139, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v115, v139, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v116, v140, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v117, v140, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v118, v141, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v119, v141, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v120, v142, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v121, v142, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v122, v143, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v123, v143, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v124, v144, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v125, v144, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v126, v145, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v127, v145, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v128, v146, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v129, v146, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v130, v147, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v131, v147, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "s_waitcnt lgkmcnt(0)\n"
        "v_fma_mix_f32 %[o], v148, v180, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v149, v180, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v150, v181, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v151, v181, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v152, v182, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v153, v182, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v154, v183, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v155, v183, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v156, v184, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v157, v184, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v158, v185, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v159, v185, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v160, v186, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v161, v186, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v162, v187, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v163, v187, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v164, v188, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v165, v188, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v166, v189, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v167, v189, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v168, v190, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v169, v190, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v170, v191, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v171, v191, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v172, v192, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v173, v192, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v174, v193, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v175, v193, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v176, v194, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v177, v194, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v178, v195, %[o] op_sel_hi:[0,1,0]\n"
        "v_fma_mix_f32 %[o], v179, v195, %[o] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
        : [o] "+v"(o), [pa] "+v"(pa), [va] "+v"(va), [nb] "+s"(nb)
        :
        : "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "v128", "v129", "v130", "v131", "v132", "v133", "v134", "v135", "v136", "v137", "v138", "v139", "v140", "v141", "v142", "v143", "v144", "v145", "v146", "v147", "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v155", "v156", "v157", "v158", "v159", "v160", "v161", "v162", "v163", "v164", "v165", "v166", "v167", "v168", "v169", "v170", "v171", "v172", "v173", "v174", "v175", "v176", "v177", "v178", "v179", "v180", "v181", "v182", "v183", "v184", "v185", "v186", "v187", "v188", "v189", "v190", "v191", "v192", "v193", "v194", "v195", "scc", "memory");
    }
    for (int j = n & ~63; j < n; j++) o = __builtin_fmaf(P[j], (float)vr[j], o);
    return o;
}

__device__ __forceinline__ float att_block_max(float v, float* red) {
    v = wave_max64(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

// byte k of a and byte k of b (int8) -> one word of two fp16, a's in the low half.
// Exact: v_perm places each byte under a 0x64 high byte, the XOR turns x into x + 128,
// so each half reads as the fp16 1024 + (x + 128), and one packed fp16 subtract of
// 1152 leaves x (integers to 2048 are exact in fp16; 0 comes out as +0).
__device__ __forceinline__ uint32_t i8x2_to_f16x2(uint32_t a, uint32_t b, int k) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t sel = (uint32_t)k | (0x0cu << 8) | ((uint32_t)(k + 4) << 16) | (0x0cu << 24);
    const uint32_t w = __builtin_amdgcn_perm(b, a, sel) ^ 0x64806480u;  // bytes 0..3 from a, 4..7 from b
    const h2 r = __builtin_bit_cast(h2, w) - (h2){(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, r);
}

// V[j0 .. j0+cnt)[d0 .. d0+ds) -> VH (fp16, [d][j] with row stride vstr halves), by
// the threads t0.. of the workgroup, key slots cnt .. cpad-1 (cpad even) written as
// zeros; each thread takes two adjacent keys so its stores are whole 32-bit words
// (adjacent lanes -> adjacent words)
__device__ __forceinline__ void att_stage_v(const int8_t* V, int hd, int d0, int ds, int j0, int cnt, int cpad,
                                            _Float16* VH, int vstr, int t0) {
    const int nthr = (int)blockDim.x - t0, t = (int)threadIdx.x - t0;
    if (t < 0) return;
    uint32_t* VW = reinterpret_cast<uint32_t*>(VH);
    const int wstr = vstr >> 1, pairs = cpad >> 1;
    if (ds == 32) {
        // 32 dims = two 16-byte pieces per key; four key pairs per thread in flight
        for (int kp0 = t; kp0 < pairs; kp0 += 4 * nthr) {
            uint4 w[4][4];  // [pair][piece of key a, piece of key b]
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int kp = kp0 + u * nthr, ja = j0 + 2 * kp;
                const bool ok = 2 * kp < cnt, hasb = 2 * kp + 1 < cnt;
                const int8_t* ra = V + (size_t)ja * hd + d0;
                w[u][0] = ok ? *reinterpret_cast<const uint4*>(ra) : make_uint4(0, 0, 0, 0);
                w[u][1] = ok ? *reinterpret_cast<const uint4*>(ra + 16) : make_uint4(0, 0, 0, 0);
                w[u][2] = hasb ? *reinterpret_cast<const uint4*>(ra + hd) : make_uint4(0, 0, 0, 0);
                w[u][3] = hasb ? *reinterpret_cast<const uint4*>(ra + hd + 16) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int kp = kp0 + u * nthr;
                if (kp < pairs) {
#pragma unroll
                    for (int pc = 0; pc < 2; pc++) {
                        const uint32_t xa[4] = {w[u][pc].x, w[u][pc].y, w[u][pc].z, w[u][pc].w};
                        const uint32_t xb[4] = {w[u][2 + pc].x, w[u][2 + pc].y, w[u][2 + pc].z, w[u][2 + pc].w};
#pragma unroll
                        for (int b = 0; b < 16; b++)
                            VW[(size_t)(pc * 16 + b) * wstr + kp] = i8x2_to_f16x2(xa[b >> 2], xb[b >> 2], b & 3);
                    }
                }
            }
        }
    } else if ((ds & 15) == 0 && ds <= 64) {
        const int pieces = ds >> 4;
        for (int kp = t; kp < pairs; kp += nthr) {
            const int ja = j0 + 2 * kp;
            const bool hasa = 2 * kp < cnt, hasb = 2 * kp + 1 < cnt;
            uint4 wa[4], wb[4];
#pragma unroll
            for (int pc = 0; pc < 4; pc++)
                if (pc < pieces) {
                    wa[pc] = hasa ? *reinterpret_cast<const uint4*>(V + (size_t)ja * hd + d0 + pc * 16)
                                  : make_uint4(0, 0, 0, 0);
                    wb[pc] = hasb ? *reinterpret_cast<const uint4*>(V + (size_t)(ja + 1) * hd + d0 + pc * 16)
                                  : make_uint4(0, 0, 0, 0);
                }
#pragma unroll
            for (int pc = 0; pc < 4; pc++)
                if (pc < pieces) {
                    const uint32_t xa[4] = {wa[pc].x, wa[pc].y, wa[pc].z, wa[pc].w};
                    const uint32_t xb[4] = {wb[pc].x, wb[pc].y, wb[pc].z, wb[pc].w};
#pragma unroll
                    for (int b = 0; b < 16; b++)
                        VW[(size_t)(pc * 16 + b) * wstr + kp] = i8x2_to_f16x2(xa[b >> 2], xb[b >> 2], b & 3);
                }
        }
    } else {  // any ds that is a multiple of 4: 4-byte words
        const int words = ds >> 2;
        for (int e = t; e < pairs * words; e += nthr) {
            const int kp = e / words, wd = e - kp * words, ja = j0 + 2 * kp;
            const uint32_t xa =
                2 * kp < cnt ? *reinterpret_cast<const uint32_t*>(V + (size_t)ja * hd + d0 + wd * 4) : 0u;
            const uint32_t xb =
                2 * kp + 1 < cnt ? *reinterpret_cast<const uint32_t*>(V + (size_t)(ja + 1) * hd + d0 + wd * 4) : 0u;
#pragma unroll
            for (int b = 0; b < 4; b++) VW[(size_t)(wd * 4 + b) * wstr + kp] = i8x2_to_f16x2(xa, xb, b);
        }
    }
}

// e_j = expf(s_j - max) for keys n0 .. n0+cnt of a long context into dst, and exact
// zeros up to the next multiple of 64, by nthr threads (t = 0 .. nthr-1), each taking
// PER keys whose scores it loads in one batch
template <int PER>
__device__ __forceinline__ void att_fill_e(float* dst, const float* S, int n0, int cnt, float mx,
                                           const uint64_t* tab, int t, int nthr) {
    const int cpad = (cnt + 63) & ~63;
    float sv[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int j = t + u * nthr;
        sv[u] = j < cnt ? S[n0 + j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int j = t + u * nthr;
        if (j < cpad) dst[j] = j < cnt ? expf_tab(sv[u] - mx, tab) : 0.0f;
    }
}

// p_j * vs_j = (e_j * (1/sum)) * vs_j for keys n0 .. n0+cnt: the loads, then (after the
// caller has issued its own) the values, zero-padded to a multiple of 64
template <int PER>
__device__ __forceinline__ void att_load_p(float* sv, float* vv, const float* S, const float* VS, int n0, int cnt,
                                           int t, int nthr) {
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int j = t + u * nthr;
        sv[u] = j < cnt ? S[n0 + j] : 0.0f;
        vv[u] = j < cnt ? VS[n0 + j] : 0.0f;
    }
}

template <int PER>
__device__ __forceinline__ void att_store_p(float* dst, const float* sv, const float* vv, int cnt, float mx,
                                            float inv, const uint64_t* tab, int t, int nthr) {
    const int cpad = (cnt + 63) & ~63;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int j = t + u * nthr;
        if (j < cpad) dst[j] = j < cnt ? (expf_tab(sv[u] - mx, tab) * inv) * vv[u] : 0.0f;
    }
}

// One long-context V chunk of a 32-dim slice: keys n0 .. n0+cnt (32 bytes of each key
// row) -> fp16 [32][ATT_LC + 8], four keys per thread (t < ATT_LC / 4), zeros to the
// next multiple of 64.  The loads go out first (att_load_v32) so the caller can issue
// its own beside them; the stores use fixed row offsets.
__device__ __forceinline__ void att_load_v32(uint4 (&w)[4][2], const int8_t* V, int hd, int d0, int n0, int cnt,
                                             int t) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int j = 4 * t + k;
        const int8_t* row = V + (size_t)(n0 + j) * hd + d0;
        w[k][0] = j < cnt ? *reinterpret_cast<const uint4*>(row) : make_uint4(0, 0, 0, 0);
        w[k][1] = j < cnt ? *reinterpret_cast<const uint4*>(row + 16) : make_uint4(0, 0, 0, 0);
    }
}

__device__ __forceinline__ void att_store_v32(const uint4 (&w)[4][2], _Float16* VH, int cnt, int t) {
    constexpr int WSTR = (ATT_LC + 8) / 2;  // words per dim row
    if (4 * t >= ((cnt + 63) & ~63)) return;
    uint32_t* base = reinterpret_cast<uint32_t*>(VH) + 2 * t;
#pragma unroll
    for (int pc = 0; pc < 2; pc++) {
        const uint32_t x[4][4] = {{w[0][pc].x, w[0][pc].y, w[0][pc].z, w[0][pc].w},
                                  {w[1][pc].x, w[1][pc].y, w[1][pc].z, w[1][pc].w},
                                  {w[2][pc].x, w[2][pc].y, w[2][pc].z, w[2][pc].w},
                                  {w[3][pc].x, w[3][pc].y, w[3][pc].z, w[3][pc].w}};
#pragma unroll
        for (int b = 0; b < 16; b++) {
            const uint32_t lo = i8x2_to_f16x2(x[0][b >> 2], x[1][b >> 2], b & 3);  // keys 4t, 4t+1
            const uint32_t hi = i8x2_to_f16x2(x[2][b >> 2], x[3][b >> 2], b & 3);  // keys 4t+2, 4t+3
            *reinterpret_cast<uint2*>(base + (pc * 16 + b) * WSTR) = make_uint2(lo, hi);
        }
    }
}

// One token's scores against every key j <= pos of its kv head, computed inside the
// softmax/PV workgroup (short contexts: one kernel for the whole attention).  Arithmetic
// as attn_scores_kernel: the token's q (and, fused, k and v) quantised by waves 0..2,
// exact int32 dots, score = (float)dot * ((ks_j * qsc) * (1/sqrt(hd))).  The key rows
// are spread over LP adjacent lanes (16 bytes each) and RB rounds of them are loaded
// in one batch.  Fused, the first workgroup of each kv head writes the new K/V slot,
// and every workgroup takes the new key from its own copy (tok8[1], toksc[1]) since
// the slot is written in this launch.  Scores go to E[0 .. pos]; ends with a barrier.
__device__ __forceinline__ void att_scores_local(const AttnArgs& a, int h, int kvh, int pos, float* E,
                                                 int8_t (&tok8)[3][256], float* toksc) {
    constexpr int RB = 12;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int hd = a.hd, nh = a.nh, nkv = a.nkv, group = nh / nkv, nk = pos + 1;
    const size_t head = (size_t)a.layer * nkv + kvh;
    const int8_t* K = a.kv.k + head * a.kv.max_seq * hd;
    const float* KS = a.kv.ks + head * a.kv.max_seq;
    const int P = hd >> 4;
    int LP = 1;
    while (LP < P) LP <<= 1;
    const int KW = 64 / LP, piece = lane & (LP - 1), kl = lane / LP;
    const bool live = piece < P;
    const int KPR = (SPV_THREADS / 64) * KW;  // keys per round
    const int R = (nk + KPR - 1) / KPR;
    const bool fused = a.fused;
    int4 kb[RB];
    float ksb[RB];
    auto issue = [&](int r0) {
#pragma unroll
        for (int u = 0; u < RB; u++) {
            const int j = (r0 + u) * KPR + wave * KW + kl;
            const bool ok = r0 + u < R && j < nk && !(fused && j == pos);
            kb[u] = ok && live ? *reinterpret_cast<const int4*>(K + (size_t)j * hd + piece * 16) : make_int4(0, 0, 0, 0);
            ksb[u] = ok ? KS[j] : 0.0f;
        }
    };
    issue(0);  // the first keys are in flight while the token's vectors are quantised
    if (fused) {
        if (wave < 3) {  // q of this head, then k, then v (kv_pack_q8, attention_q8.h:29-35)
            const float* src = wave == 0 ? a.qkv + (size_t)h * hd : a.qkv + (size_t)((wave == 1 ? nh : nh + nkv) + kvh) * hd;
            float vals[4];
            float amax = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int d = lane + 64 * c;
                vals[c] = d < hd ? src[d] : 0.0f;
                amax = fmaxf(amax, fabsf(vals[c]));
            }
            amax = wave_max64(amax);
            const float inv = quant_inv(amax);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int d = lane + 64 * c;
                if (d < hd) tok8[wave][d] = quant_i8(vals[c], inv);
            }
            if (lane == 0) toksc[wave] = quant_scale(amax);
        }
    } else {
        for (int d = tid; d < hd; d += blockDim.x) tok8[0][d] = a.q8[(size_t)h * hd + d];
        if (tid == 0) toksc[0] = a.qsc[h];
    }
    __syncthreads();
    if (fused && h % group == 0 && blockIdx.z == 0) {  // kv_pack_q8 of the new position, once per kv head
        const size_t slot = head * a.kv.max_seq + pos;
        for (int d = tid; d < hd; d += blockDim.x) {
            a.kv.k[slot * hd + d] = tok8[1][d];
            a.kv.v[slot * hd + d] = tok8[2][d];
        }
        if (tid == 0) {
            a.kv.ks[slot] = toksc[1];
            a.kv.vs[slot] = toksc[2];
        }
    }
    const float qsc = toksc[0], scale = 1.0f / sqrtf((float)hd);
    const int4 qw = live ? *reinterpret_cast<const int4*>(&tok8[0][piece * 16]) : make_int4(0, 0, 0, 0);
    const int4 knew = fused && live ? *reinterpret_cast<const int4*>(&tok8[1][piece * 16]) : make_int4(0, 0, 0, 0);
    const float ksnew = fused ? toksc[1] : 0.0f;
    for (int r0 = 0; r0 < R; r0 += RB) {
        if (r0 > 0) issue(r0);
#pragma unroll
        for (int u = 0; u < RB; u++) {
            const int j = (r0 + u) * KPR + wave * KW + kl;
            const bool here = fused && j == pos;
            const int4 k4 = here ? knew : kb[u];
            int d = __builtin_amdgcn_sdot4(qw.x, k4.x, 0, false);
            d = __builtin_amdgcn_sdot4(qw.y, k4.y, d, false);
            d = __builtin_amdgcn_sdot4(qw.z, k4.z, d, false);
            d = __builtin_amdgcn_sdot4(qw.w, k4.w, d, false);
            d = group_sum_last(d, LP);
            if (piece == LP - 1 && r0 + u < R && j < nk && j < ATT_ECAP)  // ATT_ONE <= ATT_ECAP
                E[j] = (float)d * (((here ? ksnew : ksb[u]) * qsc) * scale);
        }
    }
    __syncthreads();
}

template <bool ONE>
__global__ __launch_bounds__(SPV_THREADS) void attn_softmax_pv_kernel(AttnArgs a, int ds, int vcap, int vstr, int lc) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red[8];
    __shared__ float s_inv;
    __shared__ uint64_t exp_tab[32];
    __shared__ __align__(16) int8_t tok8[ONE ? 3 : 1][256];  // ONE: this token's q, k, v as int8
    __shared__ float toksc[3];
    float* E = reinterpret_cast<float*>(smem);                                   // [ATT_ECAP]
    _Float16* VH = reinterpret_cast<_Float16*>(smem + ATT_ECAP * sizeof(float));  // [ds][vstr]

    const int tid = threadIdx.x, wave = tid >> 6;
    const int h = blockIdx.x, rr = blockIdx.y, slice = blockIdx.z;
    const int r = a.row0 + rr;
    const int hd = a.hd, nh = a.nh, nkv = a.nkv, group = nh / nkv, kvh = h / group;
    const int pos = a.state ? a.state[0] - 1 : a.start_pos + r;
    const int nk = pos + 1;
    const int d0 = slice * ds;
    const size_t head = (size_t)a.layer * nkv + kvh;
    const int8_t* V = a.kv.v + head * a.kv.max_seq * hd;
    const float* VS = a.kv.vs + head * a.kv.max_seq;
    const float* S = a.scratch + ((size_t)rr * nh + h) * a.max_keys;

    {
        constexpr uint64_t tab[32] = JY_EXP2_TABLE;
        if (tid < 32) exp_tab[tid] = tab[tid];  // published by the barriers of the block max
    }
    if constexpr (ONE) att_scores_local(a, h, kvh, pos, E, tok8, toksc);
    // the new position's V row: from this workgroup's own copy when the kernel wrote it
    const bool vnew = ONE && a.fused;
    float o = 0.0f;
    if (ONE || nk <= ATT_ECAP) {
        // the scores and V scales of this thread's keys in one batch of loads, the max,
        // then e_j in registers and in LDS, with exact zeros up to a multiple of 64 keys
        // so the chains need no tail
        constexpr int NV = ATT_ECAP / SPV_THREADS;
        float ev[NV], vsr[NV];
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int j = tid + k * SPV_THREADS;
            ev[k] = j < nk ? (ONE ? E[j] : S[j]) : -1e30f;
            vsr[k] = j < nk ? (vnew && j == pos ? toksc[2] : VS[j]) : 0.0f;
        }
        float lmax = -1e30f;
#pragma unroll
        for (int k = 0; k < NV; k++) lmax = fmaxf(lmax, ev[k]);
        const float mx = att_block_max(lmax, red);
        const int nk64 = (nk + 63) & ~63;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int j = tid + k * SPV_THREADS;
            if (j < nk64) {
                ev[k] = j < nk ? expf_tab(ev[k] - mx, exp_tab) : 0.0f;
                E[j] = ev[k];
            }
        }
        lds_barrier();
        // the sum chain on wave 0 while the other waves stage the first run of V
        const int c0 = min(nk, vcap);
        if (tid < 16) {
            const float sum = chain_sum16(E, nk64, 0.0f);  // + 0.0 for the padding: exact
            if (tid == 0) s_inv = 1.0f / sum;
        }
        if (wave > 0) att_stage_v(V, hd, d0, ds, 0, vnew ? c0 - 1 : c0, (c0 + 63) & ~63, VH, vstr, 64);
        lds_barrier();
        const float inv = s_inv;
#pragma unroll
        for (int k = 0; k < NV; k++) {  // p_j * vs_j
            const int j = tid + k * SPV_THREADS;
            if (j < nk) E[j] = (ev[k] * inv) * vsr[k];
        }
        if (vnew && tid < ds) VH[(size_t)tid * vstr + pos] = (_Float16)(int)tok8[2][d0 + tid];  // exact
        __syncthreads();
        // the PV chain over whole 64-key blocks: the padding adds fma(0, 0, o) = o
        for (int cs = 0; cs < nk; cs += vcap) {
            const int cnt = min(vcap, nk - cs), cpad = (cnt + 63) & ~63;
            if (cs > 0) {
                __syncthreads();
                att_stage_v(V, hd, d0, ds, cs, cnt, cpad, VH, vstr, 0);
                __syncthreads();
            }
            if (tid < ds) o = chain_pv(E + cs, VH + (size_t)tid * vstr, o, cpad);
        }
    } else if constexpr (!ONE) {
        // Longer contexts.  e_j is recomputed from the scores (expf is deterministic)
        // instead of being written back: in windows of ATT_LW keys for the sum chain, and
        // again as p_j * vs_j in chunks of lc keys for the PV chain.  Each is double-
        // buffered: wave 0 runs the chain over one buffer (ds <= 64 lanes) while waves
        // 1..7 fill the other, and every hand-over is one workgroup barrier, so the
        // chains run back to back.
        float* EW = reinterpret_cast<float*>(smem);                 // [2][ATT_LW]
        float* PB = EW + 2 * ATT_LW;                                  // [2][lc], lc <= ATT_LC
        _Float16* VB = reinterpret_cast<_Float16*>(PB + 2 * lc);      // [2][ds][lc + 8]
        const int lvstr = lc + 8;
        const size_t vbuf = (size_t)ds * lvstr;
        const int pt = tid - 64;  // producer index on waves 1..7
        const bool v32 = ds == 32 && lc == ATT_LC;  // the fixed-stride V producer applies
        float lmax = -1e30f;
        {
            float lm[8];
#pragma unroll
            for (int u = 0; u < 8; u++) lm[u] = -1e30f;
            for (int j0 = tid; j0 < nk; j0 += 8 * SPV_THREADS) {
                float sv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) sv[u] = j0 + u * SPV_THREADS < nk ? S[j0 + u * SPV_THREADS] : -1e30f;
#pragma unroll
                for (int u = 0; u < 8; u++) lm[u] = fmaxf(lm[u], sv[u]);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) lmax = fmaxf(lmax, lm[u]);
        }
        const float mx = att_block_max(lmax, red);
        const int nw = (nk + ATT_LW - 1) / ATT_LW;
        att_fill_e<cdiv(ATT_LW, SPV_THREADS)>(EW, S, 0, min(ATT_LW, nk), mx, exp_tab, tid, SPV_THREADS);
        __syncthreads();
        float sum = 0.0f;
        for (int w = 0; w < nw; w++) {
            const int cnt = min(ATT_LW, nk - w * ATT_LW), cpad = (cnt + 63) & ~63;
            if (wave == 0) {
                if (tid < 16) sum = chain_sum16(EW + (w & 1) * ATT_LW, cpad, sum);  // + 0.0 padding: exact
            } else {
                if (w + 1 < nw) {
                    const int n0 = (w + 1) * ATT_LW;
                    att_fill_e<cdiv(ATT_LW, SPV_THREADS - 64)>(EW + ((w + 1) & 1) * ATT_LW, S, n0, min(ATT_LW, nk - n0),
                                                            mx, exp_tab, pt, SPV_THREADS - 64);
                }
                if (w == 0) {  // the first V chunk, while the sum chain runs
                    const int vcnt = min(lc, nk);
                    if (v32) {
                        if (pt < ATT_LC / 4) {
                            uint4 vw[4][2];
                            att_load_v32(vw, V, hd, d0, 0, vcnt, pt);
                            att_store_v32(vw, VB, vcnt, pt);
                        }
                    } else {
                        att_stage_v(V, hd, d0, ds, 0, vcnt, (vcnt + 63) & ~63, VB, lvstr, 64);
                    }
                }
            }
            __syncthreads();
        }
        if (tid == 0) s_inv = 1.0f / sum;
        __syncthreads();
        const float inv = s_inv;
        const int nc = (nk + lc - 1) / lc;
        {
            constexpr int PER = cdiv(ATT_LC, SPV_THREADS);
            float sv[PER], vv[PER];
            att_load_p<PER>(sv, vv, S, VS, 0, min(lc, nk), tid, SPV_THREADS);
            att_store_p<PER>(PB, sv, vv, min(lc, nk), mx, inv, exp_tab, tid, SPV_THREADS);
        }
        __syncthreads();
        for (int c = 0; c < nc; c++) {
            const int cnt = min(lc, nk - c * lc), cpad = (cnt + 63) & ~63;
            if (wave == 0) {
                if (tid < ds) o = chain_pv(PB + (c & 1) * lc, VB + (c & 1) * vbuf + (size_t)tid * lvstr, o, cpad);
            } else if (c + 1 < nc) {
                // the next chunk's scores, V scales and V rows in one round of loads
                const int n0 = (c + 1) * lc, ncnt = min(lc, nk - n0), npad = (ncnt + 63) & ~63;
                constexpr int PER = cdiv(ATT_LC, SPV_THREADS - 64);
                float sv[PER], vv[PER];
                att_load_p<PER>(sv, vv, S, VS, n0, ncnt, pt, SPV_THREADS - 64);
                _Float16* vh = VB + ((c + 1) & 1) * vbuf;
                if (v32) {
                    uint4 vw[4][2];
                    if (pt < ATT_LC / 4) att_load_v32(vw, V, hd, d0, n0, ncnt, pt);
                    att_store_p<PER>(PB + ((c + 1) & 1) * lc, sv, vv, ncnt, mx, inv, exp_tab, pt, SPV_THREADS - 64);
                    if (pt < ATT_LC / 4) att_store_v32(vw, vh, ncnt, pt);
                } else {
                    att_stage_v(V, hd, d0, ds, n0, ncnt, npad, vh, lvstr, 64);
                    att_store_p<PER>(PB + ((c + 1) & 1) * lc, sv, vv, ncnt, mx, inv, exp_tab, pt, SPV_THREADS - 64);
                }
            }
            __syncthreads();
        }
    }
    if (tid < ds) a.out[((size_t)r * nh + h) * hd + d0 + tid] = o;
}

// ------------------------------------------------------------------ launch

static int g_att_lds_max = 0;

// output dims per softmax/PV workgroup and the V run it stages (fp16 rows of
// vstr = vcap + 8 halves: 16 bytes of padding per row); lc: the chunk of the long-
// context form (two P chunks and two V chunks after the two e windows); lds: the
// dynamic LDS that covers both forms
static void att_shape(int hd, int* ds, int* vcap, int* vstr, int* lc, size_t* lds) {
    // 32 dims, else the largest multiple of 4 up to 64 that divides hd (hd % 4 == 0 is
    // checked at upload): the PV chain then fits in wave 0
    int d = 32;
    if (hd % 32) {
        d = 4;
        for (int c = 8; c <= 64 && c <= hd; c += 4)
            if (hd % c == 0) d = c;
    }
    *ds = d;
    const int avail = (g_att_lds_max > 0 ? g_att_lds_max : 65536) - 2048;
    const int budget = avail - ATT_ECAP * 4;
    int v = ATT_ECAP;
    while (v > 64 && (size_t)(*ds) * (v + 8) * 2 > (size_t)budget) v >>= 1;
    if (v > ATT_ECAP) v = ATT_ECAP;
    *vcap = v;
    *vstr = v + 8;
    auto long_bytes = [&](int c) { return (size_t)2 * ATT_LW * 4 + (size_t)2 * c * 4 + (size_t)2 * (*ds) * (c + 8) * 2; };
    int c = ATT_LC;  // the producers' per-thread key counts are sized for ATT_LC
    while (c > 64 && long_bytes(c) > (size_t)avail) c -= 64;
    *lc = c;
    *lds = std::max((size_t)ATT_ECAP * 4 + (size_t)(*ds) * (*vstr) * 2, long_bytes(c));
}

static int att_keys_per_wg(int hd) {
    if (hd & 15) return ATT_THREADS;
    int lp = 1;
    while (lp < (hd >> 4)) lp <<= 1;
    return (ATT_THREADS / 64) * (64 / lp) * ATT_U;
}

int att_short_keys() { return ATT_ONE; }

void launch_attention(const AttnArgs& a, hipStream_t st) {
    {
        // one token whose every replayed position attends at most ATT_ONE keys: scores,
        // softmax and PV in one kernel
        int ds, vcap, vstr, lc;
        size_t lds;
        att_shape(a.hd, &ds, &vcap, &vstr, &lc, &lds);
        const bool shortk = a.state ? a.short_ctx : a.start_pos + a.row0 + 1 <= ATT_ONE;
        if (a.nrows == 1 && (a.hd & 15) == 0 && vcap >= ATT_ECAP && shortk) {
            const size_t lds1 = (size_t)ATT_ECAP * 4 + (size_t)ds * vstr * 2;
            hipLaunchKernelGGL(attn_softmax_pv_kernel<true>, dim3(a.nh, 1, a.hd / ds), dim3(SPV_THREADS), lds1, st, a,
                               ds, vcap, vstr, lc);
            return;
        }
    }
    const int kc = att_keys_per_wg(a.hd);
    // with the position on the device (graph replays) every run up to max_keys is launched
    // and the runs past the current length return at once
    const int keys = a.state ? a.max_keys : a.start_pos + a.row0 + a.nrows;
    const int group = a.nh / a.nkv;
    const int nb = (group + ATT_GB - 1) / ATT_GB;
    hipLaunchKernelGGL(attn_scores_kernel, dim3(a.nkv * nb, (keys + kc - 1) / kc, a.nrows), dim3(ATT_THREADS), 0, st,
                       a, kc);
    int ds, vcap, vstr, lc;
    size_t lds;
    att_shape(a.hd, &ds, &vcap, &vstr, &lc, &lds);
    hipLaunchKernelGGL(attn_softmax_pv_kernel<false>, dim3(a.nh, a.nrows, a.hd / ds), dim3(SPV_THREADS), lds, st, a,
                       ds, vcap, vstr, lc);
}

hipError_t matvec_init();
hipError_t matvec_split_init();
hipError_t persist_init();
hipError_t quant_init();
hipError_t dense_init();

hipError_t kernels_init() {
    int dev = 0, mx = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return e;
    g_att_lds_max = mx;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_softmax_pv_kernel<false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, mx - 2048);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_softmax_pv_kernel<true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, mx - 2048);
    if (e != hipSuccess) return e;
    e = quant_init();
    if (e == hipSuccess) e = dense_init();
    if (e == hipSuccess) e = matvec_split_init();
    if (e == hipSuccess) e = persist_init();
    if (e == hipSuccess) e = gemm_mfma_init();
    if (e == hipSuccess) e = rope_pack_init();
    if (e != hipSuccess) return e;
    return matvec_init();
}

}  // namespace jy
