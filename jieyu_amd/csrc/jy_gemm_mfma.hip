// jy_gemm_mfma.hip — prompt (m > 1) GEMMs of Q8_0 matrices on the matrix cores, the
// tolerance mode's form of the generic matmul path (libs/matmul_libs/matmul_q.h:145-161:
// C[i][n] = sum_k A[i][k] * q[n][k] * d[n][k/32]).
//
// Numbers.  The int8 weights are exact in fp16.  Each activation row is scaled by a power
// of two that puts its largest magnitude in [2^13, 2^14) and split into an fp16 high part
// and an fp16 low part (the rounding remainder), 22 significant bits together.  One
// v_mfma_f32_16x16x32_f16 per part gives a 32-weight block's sum sum_k a[k] q[k] in fp32
// (every product exact, fp32 additions); the block's fp16 scale multiplies that sum in an
// fp32 fma into the running result, and the epilogue undoes the row's power of two.  So
// the differences from the reference's fp32 loop are the order of the fp32 additions and
// the 2^-22 relative split of the activations.
//
// Layout.  The matrix is kept a second time for these kernels (built when the mode is
// enabled): for every tile of 16 rows and every block, the 512 bytes the 64 lanes of an
// MFMA's B operand read, lane l = c + 16 G (row c of the tile, k = 8G .. 8G+7 of the
// block) holding 8 bytes; and the block scales as fp32, four blocks of a row together.
// The A operand takes lane l = r + 16 G for row r and the same k = 8G .. 8G+7: whatever
// order the instruction gives the four lane groups' k, A and B agree on it.
//
// Tiling.  A workgroup of 4 waves computes 128 rows (tokens) x 128 columns (matrix rows),
// each wave 64 x 64: 4 x 4 tiles of 16 x 16, acc in the MFMA C layout (lane l holds rows
// 4 (l/16) .. +3 of column l % 16).  Per block the workgroup stages the tile's activation
// parts and its weights (converted to fp16 once) in LDS, double-buffered, with the global
// loads two blocks ahead in registers: block b+2's loads are in flight while the waves run
// block b's MFMAs from LDS and stage block b+1.
#include "jy_layout.h"
#include "jy_mfma.h"

namespace jy {

static constexpr int GM_TILE = 128;  // workgroup tile: rows and columns

// ---------------------------------------------------------------- the matrix copy

// one thread per (16-row tile t, block b, lane l): the 8 weights of row 16t + (l % 16),
// k = 32b + 8(l/16) .. +7, from the lane-pair layout (slot r*16 + g of chunk b/8 holds
// weights 2g, 2g+1 of each of its 8 blocks at bytes 2j, 2j+1); the scales of blocks
// 4*b4 .. 4*b4+3 of each row by the threads with l < 16 and b % 4 == 0
__global__ void mfma_repack_kernel(Q8Dev W, Q8MfmaDev M) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)M.tiles * M.nb * 64;
    if (id >= total) return;
    const int l = (int)(id % 64);
    const size_t tb = id / 64;
    const int b = (int)(tb % M.nb), t = (int)(tb / M.nb);
    const int n = 16 * t + (l % 16), G = l / 16;
    uint32_t w0 = 0, w1 = 0;
    if (n < W.rows) {
        const int rg = n >> 2, r = n & 3, ch = b >> 3, j = b & 7;
        const uint8_t* chunk = W.qs + ((size_t)rg * W.nchp + ch) * 1024;
        uint32_t v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint8_t* s = chunk + (size_t)(r * 16 + 4 * G + i) * 16 + 2 * j;
            v[i] = (uint32_t)s[0] | ((uint32_t)s[1] << 8);
        }
        w0 = v[0] | (v[1] << 16);
        w1 = v[2] | (v[3] << 16);
    }
    uint2* dst = reinterpret_cast<uint2*>(M.q + (tb * 64 + l) * 8);
    *dst = make_uint2(w0, w1);
    if (l < 16 && (b & 3) == 0) {
        float4 dv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (n < W.rows) {
            const int rg = n >> 2, r = n & 3;
            float t4[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int bb = b + i;
                float s = 0.0f;
                if (bb < W.nb) {
                    const uint16_t h = W.d[((size_t)rg * W.nchp + (bb >> 3)) * 32 + r * 8 + (bb & 7)];
                    s = (float)__builtin_bit_cast(_Float16, h);
                }
                t4[i] = s;
            }
            dv = make_float4(t4[0], t4[1], t4[2], t4[3]);
        }
        reinterpret_cast<float4*>(M.d)[((size_t)t * M.nb4 + (b >> 2)) * 16 + l] = dv;
    }
}

void launch_mfma_repack(const Q8Dev& W, const Q8MfmaDev& M, hipStream_t st) {
    const size_t total = (size_t)M.tiles * M.nb * 64;
    hipLaunchKernelGGL(mfma_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, W, M);
}

// ---------------------------------------------------------------- the activation split

// one workgroup per row of the padded activations [mp][K]: rows past m are zero
__global__ __launch_bounds__(256) void mfma_split_kernel(const float* __restrict__ A, int m, int K,
                                                         _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                         float* __restrict__ unscale) {
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* a = A + (size_t)row * K;
    const bool live = row < m;
    float amax = 0.0f;
    if (live)
        for (int k = tid; k < K; k += 256) amax = fmaxf(amax, fabsf(a[k]));
    amax = wave_max64(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // 2^s with amax * 2^s in [2^13, 2^14); s kept within float's normal exponents
    int ex = 0;
    if (amax > 0.0f) frexpf(amax, &ex);
    const int s = amax > 0.0f ? min(max(14 - ex, -100), 100) : 0;
    const float up = ldexpf(1.0f, s);
    if (tid == 0) unscale[row] = ldexpf(1.0f, -s);
    _Float16* h = hi + (size_t)row * K;
    _Float16* w = lo + (size_t)row * K;
    for (int k = tid; k < K; k += 256) {
        const float v = live ? a[k] * up : 0.0f;
        const _Float16 vh = (_Float16)v;
        h[k] = vh;
        w[k] = (_Float16)(v - (float)vh);
    }
}

void launch_mfma_split(const float* A, int m, int mp, int K, _Float16* hi, _Float16* lo, float* unscale,
                       hipStream_t st) {
    hipLaunchKernelGGL(mfma_split_kernel, dim3(mp), dim3(256), 0, st, A, m, K, hi, lo, unscale);
}

// ---------------------------------------------------------------- the GEMM

// LDS of one block stage, in MFMA operand order: for each of the 8 row tiles (high and
// low parts) and 8 column tiles (weights as fp16), the 64 lanes' 16-byte operands at
// lane * 16, so that every operand read and every staging write is one contiguous 1 KiB
// per wave instruction (no bank conflicts); and the 128 columns' block scales
template <int NT>
struct GmStage {
    h8_t ah[8][64];
    h8_t al[8][64];
    h8_t bq[2 * NT][64];
    float d[32 * NT];
};

// Block b of the workgroup's tile into registers (global loads only): thread t stages
// operand positions p = t and t + 256 (row tile p/64, lane p%64: token row 16 (p/64) +
// (p%16), k 8 ((p%64)/16) .. +7) of the high and low parts; lanes 2 (t%32), +1 of column
// tile t/32 (8 weight bytes each); with t < 128 column t's scale
struct GmRegs {
    uint4 h0, h1, l0, l1;
    uint2 q0, q1;
    float d;
};

// NT column tiles per wave: a workgroup covers 128 tokens x 32 NT columns
template <int EPI, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_q8_mfma_kernel(Q8MfmaDev W, int m, int K, const _Float16* __restrict__ ahi,
                                                           const _Float16* __restrict__ alo,
                                                           const float* __restrict__ unscale, float* __restrict__ C,
                                                           int ldc, const float* __restrict__ aux) {
    __shared__ GmStage<NT> st[2];
    const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int c = l & 15, G = l >> 4;
    const int rowt = blockIdx.x * GM_TILE;               // the workgroup's first token row
    const int tilet = blockIdx.y * 2 * NT;              // its first 16-column tile
    const int nb = W.nb;

    // staging roles
    const size_t a0 = (size_t)(rowt + 16 * (tid >> 6) + c) * K + 8 * G;        // position t
    const size_t a1 = (size_t)(rowt + 16 * ((tid + 256) >> 6) + c) * K + 8 * G;  // position t + 256
    const int qt = tid >> 5, qpart = tid & 31;  // column tile (of 2 NT) and lane pair
    const bool qstage = qt < 2 * NT;
    const bool qlive = qstage && tilet + qt < W.tiles;
    const uint2* gq = reinterpret_cast<const uint2*>(W.q) + ((size_t)(qlive ? tilet + qt : 0) * nb) * 64 + 2 * qpart;
    const int dtile = tilet + (tid >> 4);
    const bool dlive = tid < 32 * NT && dtile < W.tiles;
    const float* gd = W.d + ((size_t)(dlive ? dtile : 0) * W.nb4 * 16 + (tid & 15)) * 4;

    auto fetch = [&](GmRegs& r, int b) {
        const size_t kb = (size_t)b * 32;
        r.h0 = *reinterpret_cast<const uint4*>(ahi + a0 + kb);
        r.h1 = *reinterpret_cast<const uint4*>(ahi + a1 + kb);
        r.l0 = *reinterpret_cast<const uint4*>(alo + a0 + kb);
        r.l1 = *reinterpret_cast<const uint4*>(alo + a1 + kb);
        if (qlive) {
            r.q0 = gq[(size_t)b * 64];
            r.q1 = gq[(size_t)b * 64 + 1];
        } else {
            r.q0 = r.q1 = make_uint2(0u, 0u);
        }
        r.d = dlive ? gd[(size_t)(b >> 2) * 64 + (b & 3)] : 0.0f;
    };
    auto stage = [&](const GmRegs& r, GmStage<NT>& S) {
        (&S.ah[0][0])[tid] = __builtin_bit_cast(h8_t, r.h0);
        (&S.ah[0][0])[tid + 256] = __builtin_bit_cast(h8_t, r.h1);
        (&S.al[0][0])[tid] = __builtin_bit_cast(h8_t, r.l0);
        (&S.al[0][0])[tid + 256] = __builtin_bit_cast(h8_t, r.l1);
        if (qstage) {
            S.bq[qt][2 * qpart] = q8_to_h8(r.q0.x, r.q0.y);
            S.bq[qt][2 * qpart + 1] = q8_to_h8(r.q1.x, r.q1.y);
        }
        if (tid < 32 * NT) S.d[tid] = r.d;
    };

    f4_t acc[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    bool ntv[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) ntv[nt] = tilet + wn * NT + nt < W.tiles;

    // block b's MFMAs from LDS stage b % 2
    auto compute = [&](int b) {
        const GmStage<NT>& S = st[b & 1];
        h8_t ah[4], al[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            ah[mt] = S.ah[wm * 4 + mt][l];
            al[mt] = S.al[wm * 4 + mt][l];
        }
        // two column tiles at a time: their 8 tiles' block sums (16 independent MFMAs back
        // to back), then the scaling
#pragma unroll
        for (int n0 = 0; n0 < NT; n0 += 2) {
            f4_t t[4][2];
            float dj[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const h8_t bq = S.bq[wn * NT + n0 + u][l];
                dj[u] = S.d[(wn * NT + n0 + u) * 16 + c];
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
                    t[mt][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt], bq, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const h8_t bq = S.bq[wn * NT + n0 + u][l];
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
                    t[mt][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt], bq, t[mt][u], 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[mt][n0 + u][i] = __builtin_fmaf(dj[u], t[mt][u][i], acc[mt][n0 + u][i]);
        }
    };
    // registers: ra holds the block after the one being computed (in flight since the
    // previous iteration), rb takes the loads of the block two ahead
    GmRegs ra, rb;
    fetch(ra, 0);
    if (nb > 1) fetch(rb, 1);
    stage(ra, st[0]);
    __syncthreads();
    auto iter = [&](int b, GmRegs& next, GmRegs& ahead) {
        if (b + 2 < nb) fetch(ahead, b + 2);
        compute(b);
        if (b + 1 < nb) stage(next, st[(b + 1) & 1]);
        __syncthreads();
    };
    for (int b = 0; b < nb; b += 2) {
        iter(b, rb, ra);
        if (b + 1 < nb) iter(b + 1, ra, rb);
    }

    // epilogue: acc[mt][nt][i] is C[row][col] before the row's unscale
    const int N = W.rows;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int col = 16 * (tilet + wn * NT + nt) + c;
        if (!ntv[nt] || col >= N) continue;
        const float bias = EPI == EPI_BIAS ? aux[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = rowt + wm * 64 + 16 * mt + 4 * G + i;
                if (row >= m) continue;
                const float y = acc[mt][nt][i] * unscale[row];
                float* dst = C + (size_t)row * ldc + col;
                if (EPI == EPI_RESID)
                    *dst += y;
                else
                    *dst = y + bias;
            }
    }
}

int mfma_rows_padded(int m) { return (m + GM_TILE - 1) / GM_TILE * GM_TILE; }

template <int NT>
static void gemm_mfma_launch(const Q8MfmaDev& W, int m, const _Float16* hi, const _Float16* lo, const float* unscale,
                             float* C, int ldc, const float* aux, Epi epi, hipStream_t st) {
    // x: token tiles (the fastest in dispatch order: the workgroups that read one column
    // tile's weights run together), y: column tiles
    const dim3 grid((unsigned)(mfma_rows_padded(m) / GM_TILE), (unsigned)((W.tiles + 2 * NT - 1) / (2 * NT)));
    const int K = W.nb * 32;
    switch (epi) {
        case EPI_BIAS:
            hipLaunchKernelGGL((gemm_q8_mfma_kernel<EPI_BIAS, NT>), grid, dim3(256), 0, st, W, m, K, hi, lo, unscale, C,
                               ldc, aux);
            break;
        case EPI_RESID:
            hipLaunchKernelGGL((gemm_q8_mfma_kernel<EPI_RESID, NT>), grid, dim3(256), 0, st, W, m, K, hi, lo, unscale,
                               C, ldc, aux);
            break;
        default:
            hipLaunchKernelGGL((gemm_q8_mfma_kernel<EPI_STORE, NT>), grid, dim3(256), 0, st, W, m, K, hi, lo, unscale,
                               C, ldc, aux);
            break;
    }
}

static int g_gemm_cus = 0;

// the wide tile (64 columns per wave), or the narrow one (32 columns per wave: twice the
// workgroups) when the wide tile would leave CUs with one workgroup or none (measured at
// 1024 tokens: 4096-row matrices 160 -> 154 us, 14336-column 561 -> 546 us; the 6144-row
// QKV, 384 wide workgroups, is faster wide: 185 vs 273 us)
void launch_gemm_q8_mfma(const Q8MfmaDev& W, int m, const _Float16* hi, const _Float16* lo, const float* unscale,
                         float* C, int ldc, const float* aux, Epi epi, hipStream_t st) {
    if (!g_gemm_cus) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            g_gemm_cus = cus;
        else
            g_gemm_cus = 256;
    }
    const long wide = (long)(mfma_rows_padded(m) / GM_TILE) * ((W.tiles + 7) / 8);
    if (wide > g_gemm_cus)
        gemm_mfma_launch<4>(W, m, hi, lo, unscale, C, ldc, aux, epi, st);
    else
        gemm_mfma_launch<2>(W, m, hi, lo, unscale, C, ldc, aux, epi, st);
}

}  // namespace jy
