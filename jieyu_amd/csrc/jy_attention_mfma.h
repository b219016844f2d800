// jy_attention_mfma.h — one slice of the split decode attention on the matrix cores: the
// form the separate attention kernels run (jy_attention_split.hip).  Same arithmetic
// contract as attn_slice (jy_attention_split.h): q and the token's k, v quantised to int8
// per head as kv_pack_q8 does (libs/model_libs/attention/attention_q8.h:20-37), the exact
// int32 q.k dot, score = (float)dot * ((ks * qsc) * (1/sqrtf(hd))), weights e^(score - max);
// the softmax sum and the p.v accumulation are reordered and the weights carried at 22 bits.
//
// Work split.  A workgroup of NW waves (4 or 8) takes one (kv head, slice of keys), and
// with DSP > 1 one tile of hd/DSP output dims over all the keys; wave w takes the slice's
// steps w, w+NW, ... of 32 keys and keeps its own running (max, sum, o) per query head, with
// no workgroup barrier in the key loop; the waves' results are merged through LDS at the end.
//
// One step of a wave (lane l: column c = l % 16, group g = l / 16):
//  q.k  v_mfma_i32_16x16x32_i8 per 16-key tile and 32 dims, keys as the 16 rows (A: lane l
//       holds 8 bytes of key c), query heads as the 16 columns (B).  The dims are assigned
//       to the MFMA's k positions so that lane l reads one contiguous run of hd/4 bytes of
//       its key row, dims (hd/4) g .. +hd/4 (A and B use the same assignment, the sum is
//       the same).  Columns 0..GT-1 are the group's heads and GT..2GT-1 the same heads
//       again, so lanes c and c + GT compute the same scores; the rest carry a zero query.
//       The result: lane l holds the scores of keys 4g..4g+3 (and 16+4g..16+4g+3 of the
//       second tile) for head column c.
//  softmax  per head column: the step's maximum (the lane's 8 keys, then the 4 groups),
//       and when it rises, the rescale of the sum and of o; e = exp(s - max).
//  p.v  o^T = V^T p^T on v_mfma_f32_16x16x32_f16: B = p^T is the lane's own 8 weights (key
//       k-slots 8g + e: keys 4g + e and 16 + 4g + e - 4), so the scores never leave their
//       lanes; the weight p = e * vs * 2^c (2^c: a per-wave power of two that puts the
//       largest v scale seen in [2^12, 2^13)) goes in as fp16: its rounding in columns
//       < GT, the remainder p - fp16(p) in columns GT..2GT-1, added at the end (22
//       significant bits together).  A = V^T: the V rows of the step go through the wave's
//       LDS tile, and ds_read_b64_tr_b8 hands lane l the 8 bytes V[key(g, e)][16 t + c]
//       of dim tile t; int8 -> fp16 is exact.  The result: lane l holds o^T rows (dims)
//       16 t + 4g .. +3 of head column c, the same lane layout as the softmax state.
#pragma once

#include "jy_attention_split.h"
#include "jy_mfma.h"

namespace jy {

static constexpr int MSL_STEP = 32;  // keys per step of a wave

// LDS of one slice.  Each wave's V tile and, after the keys, its o (the same bytes: a wave
// overwrites only its own tile).

// byte offset of key row r (of a step) in a wave's V tile: rows hd + 16 bytes apart, the
// second 16 keys a further 64 bytes on, so that the 8 rows one 16-lane group reads together
// for a p.v operand (keys 4g .. 4g+3 and 16+4g .. 16+4g+3) start in 8 distinct 16-byte
// bank slots (every 128 bytes wrap the LDS banks) and a row's pieces follow at +16 each
// (VW: the V bytes per key the workgroup holds, hd or one 16-dim tile; a 16-byte row needs
// no padding for that, the 64 bytes after row 16 suffice)
template <int VW>
__host__ __device__ constexpr int msl_row(int r) {
    return r * (VW + (VW >= 64 ? 16 : 0)) + 64 * (r >> 4);
}
template <int VW>
__host__ __device__ constexpr int msl_tile_bytes() {
    return msl_row<VW>(MSL_STEP - 1) + VW;
}
__host__ __device__ constexpr int msl_max(int a, int b) { return a > b ? a : b; }

template <int HD, int NW, int VW = HD>
struct MslLds {
    static constexpr int OWS = VW + 4;  // a head's o row (padded: the 8 heads' rows on distinct banks)
    static constexpr int TB = msl_max((msl_tile_bytes<VW>() + 15) / 16 * 16, SPL_GMAX * OWS * 4);
    union {
        int8_t vt[NW][TB];            // V rows of the wave's step (msl_row)
        float ow[NW][TB / 4];         // the wave's o per head column < GT: [c][dim]
    } u __attribute__((aligned(16)));
    float sc[NW][2 * MSL_STEP] __attribute__((aligned(16)));  // the step's k scales, then v scales
    int8_t q8[SPL_GMAX][HD + 16] __attribute__((aligned(16)));  // (padded: heads on distinct banks)
    int8_t knew[HD] __attribute__((aligned(16)));
    int8_t vnew[HD] __attribute__((aligned(16)));
    float qsc[SPL_GMAX];
    float mw[NW][SPL_GMAX], lw[NW][SPL_GMAX], cw[NW];
    float fw[NW][SPL_GMAX], mg[SPL_GMAX], lg[SPL_GMAX];
    float kvs_new[2];
};

// the global loads of one step: the lane's K bytes of its key in each 16-key tile, its
// pieces of the V rows, and one scale (lanes < 32: k scale of key l, others: v scale of
// key l - 32) as the raw bits of two loads, one of them out of range (zero).  The two are
// combined where the step uses them: combined where they are loaded, the OR would be
// placed at the loop's end and wait there for the loads of the steps after it.
template <int HD, int NV>
struct MslRegs {
    int4 k[2][HD / 64];
    int4 v[NV];
    unsigned ks, vs;
};

// x, or y where take
__device__ __forceinline__ int4 own_mix(int4 x, int4 y, bool take) {
    const int m = take ? -1 : 0;
    return make_int4((x.x & ~m) | (y.x & m), (x.y & ~m) | (y.y & m), (x.z & ~m) | (y.z & m), (x.w & ~m) | (y.w & m));
}

// DSP: the workgroup computes output dims VW dsl .. VW dsl + VW - 1 (VW = hd / DSP) of its
// heads; with DSP > 1 every workgroup of a kv head runs the q.k and softmax of all its keys
// (redundantly) and only its dims of p.v, so that one kernel covers the whole range without
// a merge.  PF: steps of loads a wave keeps in flight (2: the next step's loads go out a
// whole step ahead, for waves that take several steps).  RW (prompt rows only): the
// workgroup takes rows prow - RW + 1 .. prow, RW x G query columns (column c: row c / G, head
// c % G), each column's keys masked past its own row; rows below 0 are empty columns.
template <int P, int GT, int NW, bool COH, int DSP = 1, int PF = 1, int RW = 1>
__device__ __forceinline__ bool attn_slice_mfma(const AttnArgs& a, int ns, float* __restrict__ part, int kvh, int s,
                                                MslLds<P * 16, NW, P * 16 / DSP>& L, int prow = 0, int dsl = 0) {
    constexpr int HD = P * 16, ST = MSL_STEP;
    constexpr int VW = HD / DSP;  // V bytes per key this workgroup reads
    constexpr int DPL = HD / 4;   // K bytes per lane and key
    constexpr int KST = HD / 32;  // MFMA k-steps of q.k per tile
    constexpr int DT = VW / 16;   // dim tiles of p.v
    constexpr int PPK = VW / 16;  // 16-byte pieces per key row
    constexpr int KPI = 64 / PPK; // keys per V load instruction
    constexpr int NV = msl_max(1, ST * PPK / 64);  // V loads per lane and step
    constexpr bool VPART = KPI * NV > ST;          // lanes past the step's keys load no V
    static_assert(2 * GT <= 16, "head columns");
    static_assert(VW % 16 == 0 && HD % VW == 0 && PF >= 1 && PF <= 3, "shape");
    static_assert(SPL_GMAX * HD / 16 <= NW * 64, "a prompt row's query pieces: one per thread");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int nh = a.nh, nkv = a.nkv, G = nh / nkv;  // G <= GT
    const int Gc = RW * G;                           // query columns in use (<= GT)
    static_assert(RW == 1 || RW == 2 || RW == 4 || RW == 8, "rows per workgroup");
    const bool fused = a.fused;
    // (the length as loaded, no arithmetic in the branch: the wait for it then falls at its
    // first use, after the first loads)
    const int nk = a.state ? a.state[0] : a.start_pos + a.row0 + prow + 1;
    const int pos = nk - 1;
    const int chunk = split_chunk(nk, ns);
    const int j0 = s * chunk;
    // a slice past the live length: the whole workgroup leaves (slice 0 always holds keys,
    // and nothing before its first loads waits for the length)
    if (s != 0 && j0 >= nk) return false;
    const int j1 = min(nk, j0 + chunk);
    const bool holds_new = fused && (ns == 1 || j1 == nk);  // (one slice ends at the token)
    // the key taken from the workgroup's copy: only where it lies in the slice (a step of
    // the slice before may reach past its end onto it, where it is masked like any other)
    const int own = holds_new ? pos : -1;
    const size_t head = (size_t)a.layer * nkv + kvh;
    int8_t* K = a.kv.k + head * a.kv.max_seq * HD;
    int8_t* V = a.kv.v + head * a.kv.max_seq * HD;
    float* KSc = a.kv.ks + head * a.kv.max_seq;
    float* VSc = a.kv.vs + head * a.kv.max_seq;
    const float* row = a.qkv;

    // a step's global loads, in two parts so that each reuses the registers of the part of
    // the previous step already consumed: the V pieces and the scale (free once staged in
    // LDS), then the K bytes (free once the q.k MFMAs have read them).  Buffer loads whose
    // range ends at the slice's last key (a key past it reads as zeros and costs no memory
    // traffic), except the first steps of a whole range: their range is the cache's capacity,
    // so that their addresses do not wait for the live length.  A key past the slice is
    // masked in the step (no scale, no score), and the token's own key, read before it is
    // appended, is replaced there by the workgroup's copy.  A piece past the step's keys
    // gets an offset past every range (zeros).
    struct Rs {
        __amdgpu_buffer_rsrc_t k, v, ks, vs;
    };
    auto rsrc = [&](int keys) {
        return Rs{__builtin_amdgcn_make_buffer_rsrc(K, (short)0, keys * HD, 0x00020000),
                  __builtin_amdgcn_make_buffer_rsrc(V, (short)0, keys * HD, 0x00020000),
                  __builtin_amdgcn_make_buffer_rsrc(KSc, (short)0, keys * 4, 0x00020000),
                  __builtin_amdgcn_make_buffer_rsrc(VSc, (short)0, keys * 4, 0x00020000)};
    };
    const Rs rsl = rsrc(j1), rs0 = ns == 1 ? rsrc(a.kv.max_seq) : rsl;
    constexpr int FAR = 0x7ffffff0;
    auto load_vs = [&](MslRegs<HD, NV>& r, int base, const Rs& R) {
#pragma unroll
        for (int u = 0; u < NV; u++) {
            const int kr = KPI * u + lane / PPK, j = base + kr;
            const bool skip = VPART && kr >= ST;
            const i4_t x = __builtin_bit_cast(i4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                        R.v, skip ? FAR : j * HD + VW * dsl + 16 * (lane % PPK), 0, 0));
            r.v[u] = make_int4(x[0], x[1], x[2], x[3]);
        }
        const int o = 4 * (base + (lane & 31));
        // (b32 buffer loads return the raw bits)
        r.ks = __builtin_amdgcn_raw_buffer_load_b32(R.ks, lane < 32 ? o : FAR, 0, 0);
        r.vs = __builtin_amdgcn_raw_buffer_load_b32(R.vs, lane < 32 ? FAR : o, 0, 0);
    };
    auto load_k = [&](MslRegs<HD, NV>& r, int base, const Rs& R) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int j = base + 16 * t + col;
#pragma unroll
            for (int u = 0; u < HD / 64; u++) {
                const i4_t x = __builtin_bit_cast(i4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                            R.k, j * HD + DPL * grp + 16 * u, 0, 0));
                r.k[t][u] = make_int4(x[0], x[1], x[2], x[3]);
            }
        }
    };

    // the query's loads go out first, then the first step's K / V / scale loads: waits are in
    // issue order, so the quantisation below waits for the query only, with the keys in flight
    const int nitems = fused ? G + (holds_new ? 2 : 0) : 0;
    constexpr int PER = HD / 64;
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
    // prompt rows: the row's quantised query heads of this group, as the packing pass left
    // them (at most one 16-byte piece per thread), and their scales
    int4 qp = make_int4(0, 0, 0, 0);
    float qsp = 0.0f;
    // a query column's row and its (row, head) index into q8 / qsc; -1: an empty column
    auto qcol_at = [&](int cc) -> long {
        const int rr = cc / G, r = prow - (RW - 1) + rr;
        return r < 0 ? -1 : ((long)(a.row0 + r) * nh + (long)kvh * G + (cc - rr * G));
    };
    if (!fused) {
        if (tid < Gc * HD / 16) {
            const long qi = qcol_at(tid / (HD / 16));
            if (qi >= 0) qp = reinterpret_cast<const int4*>(a.q8 + (size_t)qi * HD)[tid % (HD / 16)];
        }
        if (tid < Gc) {
            const long qi = qcol_at(tid);
            if (qi >= 0) qsp = a.qsc[qi];
        }
    }
    MslRegs<HD, NV> rg[PF];  // (all masked for a wave without keys)
#pragma unroll
    for (int p = 0; p < PF; p++) {
        load_k(rg[p], j0 + ST * (wave + NW * p), rs0);
        load_vs(rg[p], j0 + ST * (wave + NW * p), rs0);
    }

    // q (and with the new position its k and v) quantised per head, as attn_slice does
#pragma unroll
    for (int t = 0; t < 3; t++) {
        const int i = wave + NW * t;
        if (i < nitems) {
            float amax = 0.0f;
#pragma unroll
            for (int c = 0; c < PER; c++) amax = fmaxf(amax, fabsf(qv[t][c]));
            amax = wave_max64(amax);
            const float inv = quant_inv(amax);
            int8_t* dst = i < G ? L.q8[i] : (i == G ? L.knew : L.vnew);
#pragma unroll
            for (int c = 0; c < PER; c++) dst[lane + 64 * c] = quant_i8(qv[t][c], inv);
            if (lane == 0) {
                if (i < G)
                    L.qsc[i] = quant_scale(amax);
                else
                    L.kvs_new[i == G ? 0 : 1] = quant_scale(amax);
            }
        }
    }
    if (!fused) {
        if (tid < Gc * HD / 16) *reinterpret_cast<int4*>(&L.q8[tid / (HD / 16)][16 * (tid % (HD / 16))]) = qp;
        if (tid < Gc) L.qsc[tid] = qsp;
    }
    for (int i = Gc * HD + tid; i < GT * HD; i += NW * 64) L.q8[i / HD][i % HD] = 0;
    if (tid < GT - Gc) L.qsc[Gc + tid] = 0.0f;
    lds_barrier();  // (the key loads stay in flight)
    if (holds_new && dsl == 0) {  // kv_pack_q8 of the new position, appended by the workgroup that holds it
        for (int d = tid; d < HD; d += NW * 64) {
            K[(size_t)pos * HD + d] = L.knew[d];
            V[(size_t)pos * HD + d] = L.vnew[d];
        }
        if (tid == 0) {
            KSc[pos] = L.kvs_new[0];
            VSc[pos] = L.kvs_new[1];
        }
    }

    // the lane's query bytes (head column col: heads col % GT in the first 2 GT columns)
    const bool qcol = col < 2 * GT;
    const int qh = col & (GT - 1);
    // (read from LDS in every step rather than held: registers are what limits the waves
    // in flight); a column past 2 GT reads head 0's bytes against a zero scale
    const int8_t* qrow8 = &L.q8[qh][DPL * grp];
    const float qsc_l = qcol ? L.qsc[qh] : 0.0f;
    const float scale = 1.0f / sqrtf((float)HD);
    const bool lo_col = col >= GT;  // carries the remainder of p

    // the tr read addresses of this lane within its wave's tile (role: row col/2 of its
    // group's 8 keys, half col%2): key 4g + (e & 3) + 16 (e >> 2) for e = col / 2
    const int tre = col >> 1;
    const int trk = 4 * grp + (tre & 3) + ((tre & 4) << 2);
    int8_t* vt = L.u.vt[wave];
    float* scw = L.sc[wave];

    f4_t acc[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) acc[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // scores are carried in log2 units (s * log2 e), so e = exp2(s - m)
    const float kq = qsc_l * (scale * 1.4426950408889634f);
    float m_run = -__builtin_inff(), l_run = 0.0f;
    float vmax = 0.0f;  // largest v scale seen
    int cexp = 0;       // its binary exponent; p is carried as p * 2^(13 - cexp)
    float pc = 8192.0f;
    bool first = true;

    // one step of the wave: keys base .. base + 31, its loads in r; r then takes the loads of
    // the step PF steps on
    auto step = [&](MslRegs<HD, NV>& cur, const int base) {
        // stage the step: V pieces into the tile, the scales; in the one step that holds
        // the token's own key, that key from the workgroup's copy (substituted by bit masks:
        // a select between an LDS load and the registers would be turned into a load through
        // a selected pointer, forcing the registers to memory)
        const bool has_own = own >= base && own < base + ST;
        float sv = __builtin_bit_cast(float, cur.ks | cur.vs);
        if (base + ST > j1 && base + (lane & 31) >= j1) sv = 0.0f;  // a key past the slice
        if (has_own) {
#pragma unroll
            for (int u = 0; u < NV; u++) {
                const int r = KPI * u + lane / PPK;
                cur.v[u] = own_mix(cur.v[u], *reinterpret_cast<const int4*>(L.vnew + VW * dsl + 16 * (lane % PPK)),
                                   base + r == own);
            }
            const int m = base + (lane & 31) == own ? -1 : 0;
            const int sn = __builtin_bit_cast(int, L.kvs_new[lane < 32 ? 0 : 1]);
            sv = __builtin_bit_cast(float, (__builtin_bit_cast(int, sv) & ~m) | (sn & m));
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const bool mine = base + 16 * t + col == own;
#pragma unroll
                for (int u = 0; u < HD / 64; u++)
                    cur.k[t][u] = own_mix(cur.k[t][u], *reinterpret_cast<const int4*>(L.knew + DPL * grp + 16 * u), mine);
            }
        }
#pragma unroll
        for (int u = 0; u < NV; u++) {
            const int r = KPI * u + lane / PPK;
            if (!VPART || r < ST) *reinterpret_cast<int4*>(vt + msl_row<VW>(r) + 16 * (lane % PPK)) = cur.v[u];
        }
        load_vs(cur, base + ST * NW * PF, rsl);  // a later step's, independent of this one's math

        // the v scales' power of two (o rescaled when the largest v scale's exponent moves),
        // then the scales into LDS: k scales, and v scales times 2^c
        const float vm = wave_max64(lane >= 32 ? sv : 0.0f);
        if (vm > vmax) {
            vmax = vm;
            const int e = __builtin_amdgcn_frexp_expf(vmax);
            if (e != cexp) {
                const int cn = min(100, max(-100, 13 - e));
                if (!first) {
                    const float f = __builtin_amdgcn_ldexpf(1.0f, cn - min(100, max(-100, 13 - cexp)));
#pragma unroll
                    for (int t = 0; t < DT; t++) acc[t] *= f;
                }
                cexp = e;
                pc = __builtin_amdgcn_ldexpf(1.0f, cn);
            }
        }
        scw[lane] = lane < 32 ? sv : sv * pc;

        // q.k: int32 dots of keys 16t + 4g + i, head column col
        i4_t d[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            d[t] = i4_t{0, 0, 0, 0};
#pragma unroll
            for (int st = 0; st < KST; st++) {
                const int4 kv4 = cur.k[t][st >> 1], qv4 = *reinterpret_cast<const int4*>(qrow8 + 16 * (st >> 1));
                const long ka = (st & 1) ? (long)(((unsigned long)(unsigned)kv4.w << 32) | (unsigned)kv4.z)
                                         : (long)(((unsigned long)(unsigned)kv4.y << 32) | (unsigned)kv4.x);
                const long qa = (st & 1) ? (long)(((unsigned long)(unsigned)qv4.w << 32) | (unsigned)qv4.z)
                                         : (long)(((unsigned long)(unsigned)qv4.y << 32) | (unsigned)qv4.x);
                d[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ka, qa, d[t], 0, 0, 0);
            }
        }
        load_k(cur, base + ST * NW * PF, rsl);
        float sc[2][4], vs[2][4];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float4 k4 = *reinterpret_cast<const float4*>(scw + 16 * t + 4 * grp);
            const float4 v4 = *reinterpret_cast<const float4*>(scw + ST + 16 * t + 4 * grp);
            sc[t][0] = (float)d[t][0] * (k4.x * kq);
            sc[t][1] = (float)d[t][1] * (k4.y * kq);
            sc[t][2] = (float)d[t][2] * (k4.z * kq);
            sc[t][3] = (float)d[t][3] * (k4.w * kq);
            vs[t][0] = v4.x;
            vs[t][1] = v4.y;
            vs[t][2] = v4.z;
            vs[t][3] = v4.w;
        }
        if (base + ST > j1) {  // a partial step: keys past the slice carry no weight
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (base + 16 * t + 4 * grp + i >= j1) sc[t][i] = -__builtin_inff();
        }
        if (RW > 1 && base + ST > j1 - (RW - 1)) {  // the keys of the group's later rows
            const int lim = j1 - (RW - 1 - qh / G);  // past the column's own row
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (base + 16 * t + 4 * grp + i >= lim) sc[t][i] = -__builtin_inff();
        }
        // the step's maximum per head column; on a rise, the rescale of what came before
        float tm = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                         fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        if (first) {
            m_run = tm;
        } else if (__any(tm > m_run)) {
            const float mn = fmaxf(m_run, tm);
            const float al = __builtin_amdgcn_exp2f(m_run - mn);
            l_run *= al;
#pragma unroll
            for (int t = 0; t < DT; t++) acc[t] *= al;
            m_run = mn;
        }
        first = false;
        // weights: e for the sum; p = e * vs * 2^c, in fp16 (columns < GT) or its remainder
        h8_t pb;
        float esum = 0.0f;
        // (with RW > 1 a column may have no key yet: its maximum is still -inf, its weights 0)
        const float mref = (RW > 1 && m_run == -__builtin_inff()) ? 0.0f : m_run;
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = __builtin_amdgcn_exp2f(sc[t][i] - mref);
                esum += e;
                const float p = e * vs[t][i];
                const _Float16 hi = (_Float16)p;
                pb[4 * t + i] = lo_col ? (_Float16)(p - (float)hi) : hi;
            }
        }
        l_run += esum;
        // p.v over the dim tiles
#pragma unroll
        for (int t = 0; t < DT; t++) {
            const i2_t vb = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (__attribute__((address_space(3))) i2_t*)(vt + msl_row<VW>(trk) + 16 * t + 8 * (col & 1)));
            const h8_t va = q8_to_h8((uint32_t)vb.x, (uint32_t)vb.y);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, acc[t], 0, 0, 0);
        }
    };
    // the wave's steps: PF at a time with no path that skips one (the compiler's wait counts
    // merge over every path into the loop head: a path with fewer loads issued would make a
    // step wait for the loads of the steps after it), then the remainder
    const int nst = j1 - j0 > ST * wave ? (j1 - j0 - ST * wave + ST * NW - 1) / (ST * NW) : 0;
    int k = 0;
    for (; k + PF <= nst; k += PF) {
#pragma unroll
        for (int p = 0; p < PF; p++) step(rg[p], j0 + ST * (wave + NW * (k + p)));
    }
#pragma unroll
    for (int p = 0; p + 1 < PF; p++)
        if (k + p < nst) step(rg[p], j0 + ST * (wave + NW * (k + p)));

    // the wave's totals: the sum over the 4 groups; o of head column c < GT plus its remainder
    // column c + GT, into the wave's tile as [c][dim] rows of OWS floats
    constexpr int OWS = MslLds<HD, NW, VW>::OWS;
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    float* ow = L.u.ow[wave];
#pragma unroll
    for (int t = 0; t < DT; t++) {
        f4_t o = acc[t];
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] += dpp_f<0x120 + (16 - GT) % 16>(o[i]);
        if (col < GT) *reinterpret_cast<f4_t*>(ow + col * OWS + 16 * t + 4 * grp) = o;
    }
    if (grp == 0 && col < GT) {
        L.mw[wave][col] = m_run;
        L.lw[wave][col] = l_run;
    }
    if (lane == 0) L.cw[wave] = __builtin_amdgcn_ldexpf(1.0f, -min(100, max(-100, 13 - cexp)));
    __syncthreads();

    // merge of the waves (log2 units): M = max m_w, factors f_w = 2^(m_w - M) 2^-c_w,
    // L = sum 2^(m_w - M) l_w, o = sum f_w o_w; M goes out in natural units.  Thread
    // (head g, wave w) = (tid / NW, tid % NW) of the first two waves (G NW <= 128), the max
    // and the sum over w as butterflies within groups of NW lanes.
    static_assert(SPL_GMAX * NW <= 128 && 64 % NW == 0, "merge lanes");
    if (tid < 128) {
        const int w = tid % NW, g = tid / NW;
        const bool ok = g < Gc;
        const float mw = ok ? L.mw[w][g] : 0.0f;
        float M = mw;
#pragma unroll
        for (int k = 1; k < NW; k <<= 1) M = fmaxf(M, __shfl_xor(M, k));
        const float f = ok ? __builtin_amdgcn_exp2f(mw - M) : 0.0f;  // 0 for a wave without keys
        float lsum = f * (ok ? L.lw[w][g] : 0.0f);
#pragma unroll
        for (int k = 1; k < NW; k <<= 1) lsum += __shfl_xor(lsum, k);
        if (ok) {
            L.fw[w][g] = f * L.cw[w];
            if (w == 0) {
                L.mg[g] = M * 0.6931471805599453f;
                L.lg[g] = lsum;
            }
        }
    }
    __syncthreads();
    const int W = HD + 2;
    for (int o = tid; o < Gc * VW; o += NW * 64) {
        const int g = o / VW, dd = o - g * VW;
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) t = __builtin_fmaf(L.fw[w][g], L.u.ow[w][g * OWS + dd], t);
        if (!part) {
            const long qi = qcol_at(g);
            if (qi >= 0) a.out[(size_t)qi * HD + VW * dsl + dd] = t / L.lg[g];
            continue;
        }
        float* out = part + ((size_t)(kvh * G + g) * ns + s) * W;
        act_st<COH>(out + dd, t);
        if (dd == 0) {
            act_st<COH>(out + HD, L.mg[g]);
            act_st<COH>(out + HD + 1, L.lg[g]);
        }
    }
    return true;
}

}  // namespace jy
