// jy_kernels.hip — CDNA4 (gfx950) kernels of jieyu's per-token decode loop.
//
// Every kernel reproduces the reference CPU arithmetic bit for bit (operation
// order and rounding), so greedy token ids match the reference exactly:
//   Q8_0 matvec        libs/matmul_libs/matmul_q.h:111-144     (32 FMA lanes, fixed tree)
//   Q8_0 prefill GEMM  libs/matmul_libs/matmul_q.h:145-161     (sequential k, mul then add)
//   f32 matvec/GEMM    libs/matmul_libs/x86/x86_classic.txt    (fma chain over k)
//   RMSNorm            libs/model_libs/rmsnorm/x86/x86_classic.txt
//   RoPE               libs/model_libs/rope/x86/x86_classic.txt
//   int8 KV / Q        libs/model_libs/attention/attention_q8.h:20-37
//   attention          libs/model_libs/attention/x86/x86_classic.txt
//   SiLU               libs/model_libs/silu/x86/x86_classic.txt
//   greedy             libs/model_libs/generate.h:57-60
#include <algorithm>

#include "jy_layout.h"

namespace jy {

// Chunks per row group are padded to a multiple of the matvec's two register
// buffers (2*U chunks), so a wave's weight stream is one linear run; U is the
// deepest of 4, 2, 1 whose padding stays within 1/16 of the row.
Q8Dev q8_shape(int rows, int cols) {
    Q8Dev q;
    q.rows = rows;
    q.cols = cols;
    q.nb = cols / 32;
    q.nch = (q.nb + 7) / 8;
    q.nbp = q.nch * 8;
    q.rows_pad = (rows + 3) / 4 * 4;
    // The register buffer depth (chunks per buffer, two buffers), which also sets the
    // zero padding of each row group to a multiple of 2U chunks.  With at least 4096
    // row groups (a full grid of waves, 16 per CU) the waves hide latency themselves:
    // the deepest buffer that needs no padding.  With fewer, each wave needs more
    // chunks in flight: four per buffer for up to 1/6 extra reads, two for up to 1/16
    // (measured at Qwen2.5-7B shapes: 3584-wide O 6.9 us at U = 4 vs 9.0 at U = 1,
    // the 37888-row gate/up 31.5 us at U = 1 vs 35.2 at U = 4).
    const bool many = q.rows_pad / 4 >= 4096;
    q.U = 1;
    for (int u : {4, 2}) {
        const int waste = (q.nch + 2 * u - 1) / (2 * u) * (2 * u) - q.nch;
        if (many ? waste == 0 : waste * (u == 4 ? 6 : 16) <= q.nch) {
            q.U = u;
            break;
        }
    }
    q.nchp = (q.nch + 2 * q.U - 1) / (2 * q.U) * (2 * q.U);
    return q;
}

// + 8 chunks of zeros after the last row group: the matvec's prefetch runs up to
// 2*U chunks past the end of a wave's run
size_t q8_qs_bytes(int rows, int cols) {
    const Q8Dev q = q8_shape(rows, cols);
    return ((size_t)(q.rows_pad / 4) * q.nchp + 8) * 1024;
}
size_t q8_d_bytes(int rows, int cols) {
    const Q8Dev q = q8_shape(rows, cols);
    return ((size_t)(q.rows_pad / 4) * q.nchp + 8) * 64;
}

// ---------------------------------------------------------------- repack

__global__ void repack_q8_kernel(const uint8_t* __restrict__ src, int rows, int nb, Q8Dev W, int row_base,
                                 int row_stride) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * nb) return;
    const int r = (int)(i / nb), b = (int)(i % nb);
    const uint8_t* s = src + i * 34;
    const int R = row_base + r * row_stride;
    const size_t chunk = q8_chunk(W, R, b >> 3);
    const int ri = R & 3, j = b & 7;
    uint8_t* q = W.qs + chunk * 1024 + (size_t)ri * 256 + j * 2;
#pragma unroll
    for (int g = 0; g < 16; g++)
        *(uint16_t*)(q + g * 16) = (uint16_t)((uint32_t)s[2 + 2 * g] | ((uint32_t)s[3 + 2 * g] << 8));
    W.d[chunk * 32 + ri * 8 + j] = (uint16_t)(s[0] | (s[1] << 8));
}

void launch_repack_q8(const uint8_t* src, int rows, int cols, const Q8Dev& dst, int row_base, int row_stride,
                      hipStream_t st) {
    const int nb = cols / 32;
    const size_t n = (size_t)rows * nb;
    hipLaunchKernelGGL(repack_q8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, rows, nb, dst,
                       row_base, row_stride);
}

// ---------------------------------------------------------------- embedding

// embedding rows (libs/model_libs/wmat_kernel.h:18-29): f32 copied, f16 converted,
// quantized rows dequantized (exact for Q8_0 and Q6_K, the one rounding of
// dequant_block for Q4_K / Q5_K).  grid (rows, ceil(hidden / 256)): one element per
// thread, so every element's loads are in flight at once
__global__ void embed_kernel(DevW E, int hidden, const int* __restrict__ ids, int id0, const int* __restrict__ state,
                             float* __restrict__ X) {
    const int i = blockIdx.x, c = blockIdx.y * blockDim.x + threadIdx.x;
    if (c >= hidden) return;
    const int id = state ? ids[state[0] - 1] : ids[id0 + i];
    const size_t e = (size_t)id * hidden + c;
    float v;
    switch (E.type) {
        case JY_F32: v = static_cast<const float*>(E.dense)[e]; break;
        case JY_F16: v = half_to_float(static_cast<const uint16_t*>(E.dense)[e]); break;
        case JY_Q8_0: v = q8_elem(E.q8, id, c); break;
        default: v = kq_elem(E.kq, id, c); break;
    }
    X[(size_t)i * hidden + c] = v;
}

void launch_embed_w(const DevW& E, int hidden, const int* ids_dev, int id_index0, const int* state, int seq,
                    float* X, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3(seq, (hidden + 255) / 256), dim3(256), 0, st, E, hidden, ids_dev,
                       id_index0, state, X);
}

void launch_embed(const Q8Dev* q8, const float* f32, int hidden, const int* ids_dev, int id_index0,
                  const int* state, int seq, float* X, hipStream_t st) {
    DevW e;
    if (q8) {
        e.type = JY_Q8_0;
        e.q8 = *q8;
    } else {
        e.type = JY_F32;
        e.dense = f32;
    }
    launch_embed_w(e, hidden, ids_dev, id_index0, state, seq, X, st);
}

// ---------------------------------------------------------------- RMSNorm

// one row per workgroup, staged in LDS, then block_rmsnorm
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ X, float* __restrict__ Y,
                                                      const float* __restrict__ w, int n) {
    extern __shared__ __align__(16) float xr[];
    __shared__ float red[18];
    const float* x = X + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) xr[i] = x[i];
    __syncthreads();
    block_rmsnorm(xr, n, w, Y + (size_t)blockIdx.x * n, red);
}

void launch_rmsnorm(const float* X, float* Y, const float* w, int n, int rows, hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), (size_t)n * sizeof(float), st, X, Y, w, n);
}

// ---------------------------------------------------------------- dense matvec (decode, [K][N] weights)

// f32 or f16 weights (an f16 weight converts to float exactly): per output an fma
// chain over k from 0 (libs/matmul_libs/x86/x86_classic.txt:2-16, matmul_f16.h:19-41).
// The chains are sequential in k, so the parallelism is one chain per output
// column.  The matrix sits in HBM as 64-column panels of 16-byte pieces
// [ceil(K/PER)][64][PER] (piece (kb, c) holds column c's rows kb*PER .. + PER - 1,
// zero past K and N), and one workgroup owns one panel: four loader waves stream
// blocks of RB rows of it (a contiguous run of pieces, plus the block's slice of x)
// into a double-buffered LDS copy of the same order while wave 0 runs the 64
// chains over the previous block, lane c reading column c's pieces (16 bytes per
// PER steps, consecutive lanes on consecutive pieces).  A zero product leaves a
// chain unchanged (it starts at +0 and never becomes -0).
__device__ __forceinline__ float dense_w(const float* B, size_t i) { return B[i]; }
__device__ __forceinline__ float dense_w(const uint16_t* B, size_t i) { return half_to_float(B[i]); }

static constexpr int DN_COLS = 64;
static constexpr int DN_THREADS = 320;  // wave 0 runs the chains, waves 1..4 load
template <typename T> struct DnShape {
    static constexpr int RB = sizeof(T) == 2 ? 512 : 256;  // rows per block (64 KiB of panel)
    static constexpr int PER = 16 / (int)sizeof(T);         // rows per 16-byte piece
    static constexpr int PIECES = RB / PER * DN_COLS;      // pieces per block
    static constexpr int LOADS = PIECES / 256;              // pieces per loader thread per block
    static constexpr size_t lds() { return (size_t)2 * PIECES * 16 + (size_t)2 * RB * sizeof(float); }
};

template <typename T>
__device__ __forceinline__ void dn_unpack(const uint4& v, T* e);
template <> __device__ __forceinline__ void dn_unpack<float>(const uint4& v, float* e) {
    e[0] = __builtin_bit_cast(float, v.x);
    e[1] = __builtin_bit_cast(float, v.y);
    e[2] = __builtin_bit_cast(float, v.z);
    e[3] = __builtin_bit_cast(float, v.w);
}
template <> __device__ __forceinline__ void dn_unpack<uint16_t>(const uint4& v, uint16_t* e) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        e[2 * i] = (uint16_t)(w[i] & 0xffffu);
        e[2 * i + 1] = (uint16_t)(w[i] >> 16);
    }
}

template <typename T, int EPI>
__global__ __launch_bounds__(DN_THREADS) void matvec_dense_kernel(const T* __restrict__ B, int K, int N,
                                                           const float* __restrict__ x, float* __restrict__ out,
                                                           const float* __restrict__ aux) {
    using S = DnShape<T>;
    constexpr int RB = S::RB, PER = S::PER, PIECES = S::PIECES, LOADS = S::LOADS;
    extern __shared__ __align__(16) unsigned char dsm[];
    uint4* tile = reinterpret_cast<uint4*>(dsm);                                  // [2][PIECES]
    float* xb = reinterpret_cast<float*>(dsm + (size_t)2 * PIECES * 16);          // [2][RB]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tid = threadIdx.x - 64;  // loader thread 0..255 (waves 1..4)
    const int j0 = blockIdx.x * DN_COLS;
    const int nkb = (K + PER - 1) / PER;
    const uint4* __restrict__ P = reinterpret_cast<const uint4*>(B) + (size_t)blockIdx.x * nkb * DN_COLS;
    const int nblk = (K + RB - 1) / RB;
    constexpr int XL = (RB + 255) / 256;  // x values per thread per block
    // two register stages: block b + 2 loads while block b + 1 waits in registers for
    // its LDS buffer and wave 0 runs the chains over block b
    uint4 v0[LOADS], v1[LOADS];
    float x0[XL], x1[XL];
    // block b's pieces into a loader thread's registers: piece e = tid + 256u of the
    // block is row piece b*RB/PER + e/64 of column e%64; rows tid, tid + 256, ... of
    // the block's x too.
    // Every load is issued (indices clamped into the panel and x; lstore puts the
    // zeros past K), so that the wait before a store leaves the later stage in flight.
    const size_t last_piece = (size_t)nkb * DN_COLS - 1;
    auto gload = [&](uint4(&v)[LOADS], float(&xv)[XL], int b) {
#pragma unroll
        for (int u = 0; u < LOADS; u++) {
            const size_t e = (size_t)b * PIECES + tid + 256 * u;
            v[u] = P[e < last_piece ? e : last_piece];
        }
#pragma unroll
        for (int i = 0; i < XL; i++) {
            const int rr = b * RB + tid + 256 * i;
            xv[i] = x[rr < K ? rr : K - 1];
        }
    };
    auto lstore = [&](const uint4(&v)[LOADS], const float(&xv)[XL], int b) {
        const int buf = b & 1;
#pragma unroll
        for (int u = 0; u < LOADS; u++) {
            const int e = tid + 256 * u;
            tile[buf * PIECES + e] = b * (RB / PER) + e / DN_COLS < nkb ? v[u] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < XL; i++) {
            const int rr = tid + 256 * i;
            if (rr < RB) xb[buf * RB + rr] = b * RB + rr < K ? xv[i] : 0.0f;
        }
    };
    float acc = 0.0f;
    // wave 0's 64 chains over block b (rows past K are zeros in LDS, so the steps run
    // to the block's last row piece rounded up to a group of G).  The LDS reads run
    // one group ahead of the fmas (two register groups, indices clamped into the
    // block so that every read is issued and each wait leaves the next group in
    // flight).
    auto chains = [&](int b) {
        if (wave != 0) return;
        constexpr int G = 4, NP = RB / PER, XQ = PER / 4;
        const int rem = nkb - b * NP;
        const int ns = rem < NP ? (rem + G - 1) / G * G : NP;
        const uint4* col = tile + (b & 1) * PIECES + lane;
        const float4* xr = reinterpret_cast<const float4*>(xb + (b & 1) * RB);
        uint4 wa[G], wb[G];
        float4 xa[G][XQ], xc[G][XQ];
        auto rd = [&](int p, uint4(&w)[G], float4(&xq)[G][XQ]) {
            p = p < NP - G ? p : NP - G;
#pragma unroll
            for (int g = 0; g < G; g++) {
                w[g] = col[(p + g) * DN_COLS];
#pragma unroll
                for (int q = 0; q < XQ; q++) xq[g][q] = xr[(p + g) * XQ + q];
            }
        };
        auto fm = [&](const uint4(&w)[G], const float4(&xq)[G][XQ]) {
#pragma unroll
            for (int g = 0; g < G; g++) {
                T el[PER];
                dn_unpack<T>(w[g], el);
                float xs[PER];
                __builtin_memcpy(xs, xq[g], sizeof(xs));
#pragma unroll
                for (int k = 0; k < PER; k++) acc = __builtin_fmaf(xs[k], dense_w(el, k), acc);
            }
        };
        rd(0, wa, xa);
        for (int p = 0; p < ns; p += 2 * G) {
            rd(p + G, wb, xc);
            __builtin_amdgcn_sched_barrier(0);  // keep the next group's reads ahead of the fmas
            fm(wa, xa);
            rd(p + 2 * G, wa, xa);
            __builtin_amdgcn_sched_barrier(0);
            if (p + G < ns) fm(wb, xc);
        }
    };
    // Phase b + 1 (between barriers b and b + 1, b = 0 .. nblk - 1): wave 0 runs the
    // chains over block b in LDS buffer b & 1 while the loaders, holding block b + 1 in
    // registers, issue the loads of block b + 2 into the other register set and then
    // store block b + 1 into buffer (b + 1) & 1, which the chains left in phase b.
    // Each side passes 1 + nblk barriers.
    if (wave == 0) {
        __syncthreads();
        for (int b = 0; b < nblk; b++) {
            chains(b);
            __syncthreads();
        }
    } else {
        gload(v0, x0, 0);
        gload(v1, x1, nblk > 1 ? 1 : 0);
        lstore(v0, x0, 0);
        __syncthreads();
        for (int b = 0; b < nblk; b += 2) {
            gload(v0, x0, b + 2 < nblk ? b + 2 : nblk - 1);  // past the end: a re-read, never stored
            if (b + 1 < nblk) lstore(v1, x1, b + 1);
            __syncthreads();
            if (b + 1 < nblk) {
                gload(v1, x1, b + 3 < nblk ? b + 3 : nblk - 1);
                if (b + 2 < nblk) lstore(v0, x0, b + 2);
                __syncthreads();
            }
        }
    }
    const int j = j0 + lane;
    if (wave == 0 && j < N) {
        if (EPI == EPI_STORE) out[j] = acc;
        if (EPI == EPI_BIAS) out[j] = acc + aux[j];
        if (EPI == EPI_RESID) out[j] = out[j] + acc;
        if (EPI == EPI_SWIGLU) out[j] = silu_at(aux[j], j, N) * acc;  // aux: the gate row; acc: up
    }
}

template <typename T>
static void matvec_dense(const T* B, int K, int N, const float* x, float* out, const float* aux, Epi epi,
                         hipStream_t st) {
    const dim3 grid((unsigned)((N + DN_COLS - 1) / DN_COLS)), block(DN_THREADS);
    const size_t lds = DnShape<T>::lds();
    switch (epi) {
    case EPI_STORE:
        hipLaunchKernelGGL((matvec_dense_kernel<T, EPI_STORE>), grid, block, lds, st, B, K, N, x, out, aux);
        break;
    case EPI_BIAS:
        hipLaunchKernelGGL((matvec_dense_kernel<T, EPI_BIAS>), grid, block, lds, st, B, K, N, x, out, aux);
        break;
    case EPI_RESID:
        hipLaunchKernelGGL((matvec_dense_kernel<T, EPI_RESID>), grid, block, lds, st, B, K, N, x, out, aux);
        break;
    case EPI_SWIGLU:
        hipLaunchKernelGGL((matvec_dense_kernel<T, EPI_SWIGLU>), grid, block, lds, st, B, K, N, x, out, aux);
        break;
    default: break;
    }
}

void launch_matvec_f32(const float* B, int K, int N, const float* x, float* out, const float* aux, Epi epi,
                       hipStream_t st) {
    matvec_dense<float>(B, K, N, x, out, aux, epi, st);
}

void launch_matvec_f16(const uint16_t* B, int K, int N, const float* x, float* out, const float* aux, Epi epi,
                       hipStream_t st) {
    matvec_dense<uint16_t>(B, K, N, x, out, aux, epi, st);
}

template <typename T>
static hipError_t dense_attr() {
    hipError_t e = hipSuccess;
    for (const void* f : {reinterpret_cast<const void*>(&matvec_dense_kernel<T, EPI_STORE>),
                          reinterpret_cast<const void*>(&matvec_dense_kernel<T, EPI_BIAS>),
                          reinterpret_cast<const void*>(&matvec_dense_kernel<T, EPI_RESID>),
                          reinterpret_cast<const void*>(&matvec_dense_kernel<T, EPI_SWIGLU>)})
        if (e == hipSuccess)
            e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)DnShape<T>::lds());
    return e;
}

hipError_t dense_init() {
    const hipError_t a = dense_attr<float>(), b = dense_attr<uint16_t>();
    return a != hipSuccess ? a : b;
}

// ---------------------------------------------------------------- prefill GEMMs (m > 1)

// 64 tokens x 64 output rows per workgroup, 4x4 outputs per thread, k in order.
// Quantized weights: acc = acc + x*w, rounded separately (the generic path of
// matmul_q, libs/matmul_libs/matmul_q.h:145-161); the weight accessor dequantizes
// exactly as dequant_block does.
struct Q8Acc {
    Q8Dev W;
    __device__ float operator()(int R, int k) const { return q8_elem(W, R, k); }
};
struct KQAcc {
    KQDev W;
    __device__ float operator()(int R, int k) const { return kq_elem(W, R, k); }
};

template <class Acc, int EPI>
__global__ __launch_bounds__(256) void gemm_quant_kernel(Acc W, int K, int N, int m, const float* __restrict__ A,
                                                         float* __restrict__ Cm, int ldc,
                                                         const float* __restrict__ aux) {
    __shared__ float xs[32][68];
    __shared__ float ws[32][68];
    const int t = threadIdx.x, ti = t & 15, tj = t >> 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = 0.0f;
    const int lt = t >> 2, lc = (t & 3) * 8;  // loader: token/row lt, k offset lc
    for (int k0 = 0; k0 < K; k0 += 32) {
        {
            const int tok = m0 + lt;
#pragma unroll
            for (int c = 0; c < 8; c++) xs[lc + c][lt] = tok < m ? A[(size_t)tok * K + k0 + lc + c] : 0.0f;
            const int R = n0 + lt;
#pragma unroll
            for (int c = 0; c < 8; c++) ws[lc + c][lt] = R < N ? W(R, k0 + lc + c) : 0.0f;
        }
        __syncthreads();
#pragma unroll 4
        for (int kk = 0; kk < 32; kk++) {
            const float4 xv = *reinterpret_cast<const float4*>(&xs[kk][ti * 4]);
            const float4 wv = *reinterpret_cast<const float4*>(&ws[kk][tj * 4]);
            const float xa[4] = {xv.x, xv.y, xv.z, xv.w}, wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) acc[a][b] = __fadd_rn(acc[a][b], __fmul_rn(xa[a], wa[b]));
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int i = m0 + ti * 4 + a;
        if (i >= m) continue;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int j = n0 + tj * 4 + b;
            if (j >= N) continue;
            float* c = Cm + (size_t)i * ldc + j;
            if (EPI == EPI_STORE) *c = acc[a][b];
            if (EPI == EPI_BIAS) *c = acc[a][b] + aux[j];
            if (EPI == EPI_RESID) *c = *c + acc[a][b];
        }
    }
}

// dense [K][N] in the panel layout (f32, or f16 converted exactly): C = fma(A[i][p],
// B[p][j], C) in order of p.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_dense_kernel(const T* __restrict__ B, int K, int N, int m,
                                                         const float* __restrict__ A, float* __restrict__ Cm, int ldc,
                                                         const float* __restrict__ aux) {
    __shared__ float xs[32][68];
    __shared__ float ws[32][68];
    const int t = threadIdx.x, ti = t & 15, tj = t >> 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = 0.0f;
    const int lt = t >> 2, lc = (t & 3) * 8;
    for (int k0 = 0; k0 < K; k0 += 32) {
        const int tok = m0 + lt;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int k = k0 + lc + c;
            xs[lc + c][lt] = (tok < m && k < K) ? A[(size_t)tok * K + k] : 0.0f;
        }
        // B rows k0..k0+31, columns n0..n0+63 of panel blockIdx.x: (32 / PER) x 64
        // 16-byte pieces, piece pc = row piece pc / 64 of column pc % 64 (zeros past K
        // come from the panel's padding; pieces past it are not read)
        {
            constexpr int PER = 16 / (int)sizeof(T), NPC = 32 / PER * 64 / 256;
            const int nkb = (K + PER - 1) / PER;
            const uint4* Pn = reinterpret_cast<const uint4*>(B) + (size_t)blockIdx.x * nkb * 64;
#pragma unroll
            for (int i = 0; i < NPC; i++) {
                const int pc = t + 256 * i, kb = k0 / PER + pc / 64, col = pc % 64;
                T el[PER];
                if (kb < nkb) {
                    dn_unpack<T>(Pn[(size_t)kb * 64 + col], el);
                } else {
#pragma unroll
                    for (int u = 0; u < PER; u++) el[u] = (T)0;
                }
#pragma unroll
                for (int u = 0; u < PER; u++) ws[(pc / 64) * PER + u][col] = dense_w(el, u);
            }
        }
        __syncthreads();
        const int kmax = K - k0 < 32 ? K - k0 : 32;
        for (int kk = 0; kk < kmax; kk++) {
            const float4 xv = *reinterpret_cast<const float4*>(&xs[kk][ti * 4]);
            const float4 wv = *reinterpret_cast<const float4*>(&ws[kk][tj * 4]);
            const float xa[4] = {xv.x, xv.y, xv.z, xv.w}, wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) acc[a][b] = __builtin_fmaf(xa[a], wa[b], acc[a][b]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int i = m0 + ti * 4 + a;
        if (i >= m) continue;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int j = n0 + tj * 4 + b;
            if (j >= N) continue;
            float* c = Cm + (size_t)i * ldc + j;
            if (EPI == EPI_STORE) *c = acc[a][b];
            if (EPI == EPI_BIAS) *c = acc[a][b] + aux[j];
            if (EPI == EPI_RESID) *c = *c + acc[a][b];
        }
    }
}

template <class Acc>
static void gemm_quant(const Acc& W, int K, int N, int m, const float* A, float* C, int ldc, const float* aux,
                       Epi epi, hipStream_t st) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((m + 63) / 64)), block(256);
    if (epi == EPI_STORE)
        hipLaunchKernelGGL((gemm_quant_kernel<Acc, EPI_STORE>), grid, block, 0, st, W, K, N, m, A, C, ldc, aux);
    if (epi == EPI_BIAS)
        hipLaunchKernelGGL((gemm_quant_kernel<Acc, EPI_BIAS>), grid, block, 0, st, W, K, N, m, A, C, ldc, aux);
    if (epi == EPI_RESID)
        hipLaunchKernelGGL((gemm_quant_kernel<Acc, EPI_RESID>), grid, block, 0, st, W, K, N, m, A, C, ldc, aux);
}

template <typename T>
static void gemm_dense(const T* B, int K, int N, int m, const float* A, float* C, int ldc, const float* aux, Epi epi,
                       hipStream_t st) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((m + 63) / 64)), block(256);
    if (epi == EPI_STORE)
        hipLaunchKernelGGL((gemm_dense_kernel<T, EPI_STORE>), grid, block, 0, st, B, K, N, m, A, C, ldc, aux);
    if (epi == EPI_BIAS)
        hipLaunchKernelGGL((gemm_dense_kernel<T, EPI_BIAS>), grid, block, 0, st, B, K, N, m, A, C, ldc, aux);
    if (epi == EPI_RESID)
        hipLaunchKernelGGL((gemm_dense_kernel<T, EPI_RESID>), grid, block, 0, st, B, K, N, m, A, C, ldc, aux);
}

void launch_gemm_q8(const Q8Dev& W, int m, const float* A, float* C, const float* aux, Epi epi, hipStream_t st) {
    gemm_quant(Q8Acc{W}, W.cols, W.rows, m, A, C, W.rows, aux, epi, st);
}

void launch_gemm_f32(const float* B, int K, int N, int m, const float* A, float* C, const float* aux, Epi epi,
                     hipStream_t st) {
    gemm_dense<float>(B, K, N, m, A, C, N, aux, epi, st);
}

void launch_gemm(const DevW& W, int m, const float* A, float* C, int ldc, const float* aux, Epi epi,
                 hipStream_t st) {
    switch (W.type) {
        case JY_F32: gemm_dense(static_cast<const float*>(W.dense), W.in, W.out, m, A, C, ldc, aux, epi, st); break;
        case JY_F16: gemm_dense(static_cast<const uint16_t*>(W.dense), W.in, W.out, m, A, C, ldc, aux, epi, st); break;
        case JY_Q8_0: gemm_quant(Q8Acc{W.q8}, W.in, W.out, m, A, C, ldc, aux, epi, st); break;
        default: gemm_quant(KQAcc{W.kq}, W.in, W.out, m, A, C, ldc, aux, epi, st); break;
    }
}

__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, int interleaved, int m,
                                int F, float* __restrict__ h) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (size_t)m * F) return;
    const size_t i = e / F, j = e % F;
    const float gv = interleaved ? g[i * 2 * F + 2 * j] : g[e];
    const float uv = interleaved ? g[i * 2 * F + 2 * j + 1] : u[e];
    h[e] = silu_at(gv, e, (size_t)m * F) * uv;
}

void launch_silu_mul(const float* g, const float* u, int interleaved, int m, int F, float* h, hipStream_t st) {
    const size_t n = (size_t)m * F;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, interleaved, m, F, h);
}

// ---------------------------------------------------------------- RoPE + int8 packing

__device__ __forceinline__ float wave_max(float v) { return wave_max64(v); }

// One workgroup per token row.  Rotation of pair m of a head uses the table row of
// position pos; within every full group of 8 pairs the reference's store order puts
// rotated pairs (4,5) in slots (2,3) and pairs (2,3) in slots (4,5)
// (rope/x86/x86_classic.txt:23-29); remainder pairs stay in place.  Then K (after
// RoPE) and V are packed into the cache and Q is quantised per head.  The rotated q / k
// go to LDS (sm) and are quantised from there; nothing is written back to qkv.  With
// kz > 1 the row is first added up into LDS (raw) from the kz partial sums
// [z][rows][width] a GEMM split over K left (in slice order, then the bias: the sum
// kernel's arithmetic) and read from there instead of qkv.
__global__ __launch_bounds__(256) void rope_pack_kernel(const float* __restrict__ qkv, int start_pos,
                                                        const int* __restrict__ state, int nh, int nkv, int hd,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, KVDev kv, int layer,
                                                        int8_t* __restrict__ q8, float* __restrict__ qsc,
                                                        const float* __restrict__ kp, int kz, int rows,
                                                        const float* __restrict__ bias) {
    extern __shared__ __align__(16) float sm[];
    const int row = blockIdx.x;
    const int pos = state ? state[0] - 1 : start_pos + row;
    const int half = hd / 2, qd = nh * hd, kvd = nkv * hd, width = qd + 2 * kvd;
    float* raw = sm + (size_t)(nh + nkv) * hd;
    const float* src_row = qkv + (size_t)row * width;
    if (kz > 1) {
        const size_t mn = (size_t)rows * width;
        for (int e = threadIdx.x; e < width; e += blockDim.x) {
            const size_t i = (size_t)row * width + e;
            float y = kp[i];
            for (int z = 1; z < kz; z++) y += kp[(size_t)z * mn + i];
            raw[e] = bias ? y + bias[e] : y;
        }
        __syncthreads();
        src_row = raw;
    }
    const float* c = cos_t + (size_t)pos * half;
    const float* s = sin_t + (size_t)pos * half;
    const int npairs = (nh + nkv) * half;
    const int full = half / 8 * 8;
    for (int e = threadIdx.x; e < npairs; e += blockDim.x) {
        const int hh = e / half, m = e - hh * half;
        const float* xh = src_row + (size_t)hh * hd;
        const float x0 = xh[2 * m], x1 = xh[2 * m + 1];
        const float cm = c[m], sn = s[m];
        const float y0 = __builtin_fmaf(x0, cm, -(x1 * sn));
        const float y1 = __builtin_fmaf(x0, sn, x1 * cm);
        int dst = m;
        if (m < full) {
            const int o = m & 7;
            dst = m - o + ((o == 2 || o == 3) ? o + 2 : (o == 4 || o == 5) ? o - 2 : o);
        }
        sm[hh * hd + 2 * dst] = y0;
        sm[hh * hd + 2 * dst + 1] = y1;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int hh = wave; hh < nh + 2 * nkv; hh += nw) {
        const float* src = (hh < nh + nkv ? sm : src_row) + (size_t)hh * hd;  // q, k rotated; v as it is
        float amax = 0.0f;
        for (int d = lane; d < hd; d += 64) amax = fmaxf(amax, fabsf(src[d]));
        amax = wave_max(amax);
        const float inv = quant_inv(amax), scl = quant_scale(amax);
        int8_t* dst;
        float* sdst;
        if (hh < nh) {
            dst = q8 + ((size_t)row * nh + hh) * hd;
            sdst = qsc + (size_t)row * nh + hh;
        } else {
            const bool isv = hh >= nh + nkv;
            const int kh = hh - nh - (isv ? nkv : 0);
            const size_t slot = ((size_t)layer * nkv + kh) * kv.max_seq + pos;
            dst = (isv ? kv.v : kv.k) + slot * hd;
            sdst = (isv ? kv.vs : kv.ks) + slot;
        }
        for (int d = lane; d < hd; d += 64) dst[d] = quant_i8(src[d], inv);
        if (lane == 0) *sdst = scl;
    }
}

// The same with the row in registers (NV float4s per thread, rows of at most 1024 NV floats):
// the table entries and then every load of the row (or of its kz partial sums) go out at once,
// the rotated q / k pairs go to their slots in LDS as float4s, the v heads beside them, and
// each head is quantised from LDS with 2-byte stores.  Every value is computed as in
// rope_pack_kernel (the same operations in the same order), so the bytes are the same.
template <int NV>
__global__ __launch_bounds__(256) void rope_pack4_kernel(const float* __restrict__ qkv, int start_pos,
                                                         const int* __restrict__ state, int nh, int nkv, int hd,
                                                         const float* __restrict__ cos_t,
                                                         const float* __restrict__ sin_t, KVDev kv, int layer,
                                                         int8_t* __restrict__ q8, float* __restrict__ qsc,
                                                         const float* __restrict__ kp, int kz, int rows,
                                                         const float* __restrict__ bias) {
    extern __shared__ __align__(16) float sm[];  // the row after RoPE: q, k rotated, v as it is
    const int row = blockIdx.x, tid = threadIdx.x;
    const int pos = state ? state[0] - 1 : start_pos + row;
    const int half = hd / 2, width = (nh + 2 * nkv) * hd, w4 = width / 4, rot = (nh + nkv) * hd;
    const int full = half / 8 * 8;
    const float* c = cos_t + (size_t)pos * half;
    const float* s = sin_t + (size_t)pos * half;
    // head of element e (a shift where hd is a power of two: no integer division)
    const int hsh = (hd & (hd - 1)) == 0 ? __builtin_ctz(hd) : -1;
    auto head_of = [&](int e) { return hsh >= 0 ? e >> hsh : e / hd; };
    // the table entries of the thread's pairs (m0, m0 + 1: m0 = (4 k4 mod hd) / 2, even)
    float2 cm[NV], sn[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int e = 4 * (tid + 256 * j), m0 = (e - head_of(e) * hd) / 2;
        const bool r = e < rot;
        cm[j] = r ? *reinterpret_cast<const float2*>(c + m0) : make_float2(0.0f, 0.0f);
        sn[j] = r ? *reinterpret_cast<const float2*>(s + m0) : make_float2(0.0f, 0.0f);
    }
    float4 v[NV];
    if (kz > 1) {  // the sum kernel's order: the slices, then the bias
        const size_t mn4 = (size_t)rows * w4;
        const float4* p4 = reinterpret_cast<const float4*>(kp) + (size_t)row * w4;
        const float4* b4 = reinterpret_cast<const float4*>(bias);
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int k4 = tid + 256 * j;
            if (k4 >= w4) break;
            float4 y = p4[k4];
            for (int z = 1; z < kz; z++) {
                const float4 t = p4[(size_t)z * mn4 + k4];
                y = make_float4(y.x + t.x, y.y + t.y, y.z + t.z, y.w + t.w);
            }
            if (bias) {
                const float4 b = b4[k4];
                y = make_float4(y.x + b.x, y.y + b.y, y.z + b.z, y.w + b.w);
            }
            v[j] = y;
        }
    } else {
        const float4* src4 = reinterpret_cast<const float4*>(qkv + (size_t)row * width);
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int k4 = tid + 256 * j;
            v[j] = k4 < w4 ? src4[k4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k4 = tid + 256 * j, e = 4 * k4;
        if (k4 >= w4) break;
        const float4 x = v[j];
        if (e < rot) {
            const int hh = head_of(e), m0 = (e - hh * hd) / 2;
            float4 y;
            y.x = __builtin_fmaf(x.x, cm[j].x, -(x.y * sn[j].x));
            y.y = __builtin_fmaf(x.x, sn[j].x, x.y * cm[j].x);
            y.z = __builtin_fmaf(x.z, cm[j].y, -(x.w * sn[j].y));
            y.w = __builtin_fmaf(x.z, sn[j].y, x.w * cm[j].y);
            int dst = m0;  // (pairs 2, 3 of a group of 8 to slots 4, 5 and back; m0 + 1 follows m0)
            if (m0 < full) {
                const int o = m0 & 7;
                dst = m0 - o + (o == 2 ? 4 : o == 4 ? 2 : o);
            }
            *reinterpret_cast<float4*>(sm + hh * hd + 2 * dst) = y;
        } else {
            *reinterpret_cast<float4*>(sm + e) = x;
        }
    }
    __syncthreads();
    const int lane = tid & 63, wave = tid >> 6, nhead = nh + 2 * nkv;
    // where head hh's bytes and scale go: q8 / qsc, or the K / V cache slot of this position
    auto target = [&](int hh, int8_t*& dst, float*& sdst) {
        if (hh < nh) {
            dst = q8 + ((size_t)row * nh + hh) * hd;
            sdst = qsc + (size_t)row * nh + hh;
        } else {
            const bool isv = hh >= nh + nkv;
            const int kh = hh - nh - (isv ? nkv : 0);
            const size_t slot = ((size_t)layer * nkv + kh) * kv.max_seq + pos;
            dst = (isv ? kv.v : kv.k) + slot * hd;
            sdst = (isv ? kv.vs : kv.ks) + slot;
        }
    };
    const int lg = hd / 4;  // lanes per head at 4 values a lane
    if (lg <= 64 && (lg & (lg - 1)) == 0) {
        // 64 / lg heads per wave: the group's maximum by xor exchanges within the group
        const int hpw = 64 / lg, gi = lane / lg, gl = lane - gi * lg;
        for (int h0 = wave * hpw; h0 < nhead; h0 += 4 * hpw) {
            const int hh = h0 + gi;
            const bool on = hh < nhead;
            const float4 x = on ? *reinterpret_cast<const float4*>(sm + (size_t)hh * hd + 4 * gl)
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float amax = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
            for (int o = 1; o < lg; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
            if (!on) continue;
            const float inv = quant_inv(amax);
            int8_t* dst;
            float* sdst;
            target(hh, dst, sdst);
            const uint32_t b0 = (uint8_t)quant_i8(x.x, inv), b1 = (uint8_t)quant_i8(x.y, inv);
            const uint32_t b2 = (uint8_t)quant_i8(x.z, inv), b3 = (uint8_t)quant_i8(x.w, inv);
            *reinterpret_cast<uint32_t*>(dst + 4 * gl) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            if (gl == 0) *sdst = quant_scale(amax);
        }
        return;
    }
    // other head sizes: wave w quantises heads w, w + 4, ... (lane l values l, l + 64, ...)
    for (int hh = wave; hh < nhead; hh += 4) {
        const float* src = sm + (size_t)hh * hd;
        float amax = 0.0f;
        for (int d = lane; d < hd; d += 64) amax = fmaxf(amax, fabsf(src[d]));
        amax = wave_max(amax);
        const float inv = quant_inv(amax);
        int8_t* dst;
        float* sdst;
        target(hh, dst, sdst);
        for (int d = lane; d < hd; d += 64) dst[d] = quant_i8(src[d], inv);
        if (lane == 0) *sdst = quant_scale(amax);
    }
}

hipError_t rope_pack_init() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&rope_pack_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                               160 * 1024 - 2048);
}

void launch_rope_pack(const float* qkv, int seq, int start_pos, const int* state, int nh, int nkv, int hd,
                      const float* cos_t, const float* sin_t, const KVDev& kv, int layer, int8_t* q8, float* qsc,
                      hipStream_t st, const float* kp, int kz, const float* bias) {
    const int width = (nh + 2 * nkv) * hd;  // (hd is a multiple of 4)
    const size_t lds4 = (size_t)width * sizeof(float);
#define JY_ROPE4(NV)                                                                                                \
    hipLaunchKernelGGL(rope_pack4_kernel<NV>, dim3(seq), dim3(256), lds4, st, qkv, start_pos, state, nh, nkv, hd, \
                       cos_t, sin_t, kv, layer, q8, qsc, kp, kz, seq, bias)
    if (width <= 1024)
        JY_ROPE4(1);
    else if (width <= 2048)
        JY_ROPE4(2);
    else if (width <= 4096)
        JY_ROPE4(4);
    else if (width <= 8192)
        JY_ROPE4(8);
    else {
        const size_t lds = (size_t)(kz > 1 ? 2 * nh + 3 * nkv : nh + nkv) * hd * sizeof(float);
        hipLaunchKernelGGL(rope_pack_kernel, dim3(seq), dim3(256), lds, st, qkv, start_pos, state, nh, nkv, hd, cos_t,
                           sin_t, kv, layer, q8, qsc, kp, kz, seq, bias);
    }
#undef JY_ROPE4
}

// ---------------------------------------------------------------- greedy selection

// next = first index of the strict maximum (generate.h:57-60); repetition penalty
// first, applied once per occurrence in generation order (generate.h:50-56): ids
// are split across threads by value, so each id's occurrences stay in order.
__global__ __launch_bounds__(1024) void argmax_kernel(float* __restrict__ logits, int V, int* __restrict__ ids,
                                                      int* __restrict__ state, const int* __restrict__ eos,
                                                      int neos, float rp, int prompt_len) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int t = threadIdx.x;
    const int len = state[0];
    if (rp != 1.0f) {
        for (int i = prompt_len; i < len; i++) {
            const int id = ids[i];
            if (id >= 0 && id < V && (id & 1023) == t) {
                const float l = logits[id];
                logits[id] = l > 0.0f ? l / rp : l * rp;
            }
        }
        __syncthreads();
    }
    float best = -__builtin_inff();
    int bidx = 0x7fffffff;
    for (int v = t; v < V; v += blockDim.x) {
        const float l = logits[v];
        if (l > best || bidx == 0x7fffffff) {
            if (!(l <= best)) {
                best = l;
                bidx = v;
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(bidx, o);
        if (ov > best || (ov == best && oi < bidx)) {
            best = ov;
            bidx = oi;
        }
    }
    if ((t & 63) == 0) {
        bv[t >> 6] = best;
        bi[t >> 6] = bidx;
    }
    __syncthreads();
    if (t == 0) {
        best = bv[0];
        bidx = bi[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++)
            if (bv[w] > best || (bv[w] == best && bi[w] < bidx)) {
                best = bv[w];
                bidx = bi[w];
            }
        if (bidx == 0x7fffffff) bidx = 0;
        if (!state[1]) {
            ids[len] = bidx;
            state[0] = len + 1;
            for (int e = 0; e < neos; e++)
                if (bidx == eos[e]) state[1] = 1;
        }
    }
}

void launch_argmax(const float* logits, int V, int* ids, int* state, const int* eos, int neos, float rep_penalty,
                   int prompt_len, hipStream_t st) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, st, const_cast<float*>(logits), V, ids, state, eos, neos,
                       rep_penalty, prompt_len);
}

// ---------------------------------------------------------------- KV layout conversion

__global__ void kv_import_kernel(const int8_t* __restrict__ k_ref, const float* __restrict__ ks_ref,
                                 const int8_t* __restrict__ v_ref, const float* __restrict__ vs_ref, int pos0,
                                 int npos, KVDev kv, int layer) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per = (size_t)kv.nkv * kv.hd;
    if (e >= (size_t)npos * per) return;
    const int p = (int)(e / per), rem = (int)(e % per), h = rem / kv.hd, d = rem % kv.hd;
    const size_t slot = ((size_t)layer * kv.nkv + h) * kv.max_seq + pos0 + p;
    kv.k[slot * kv.hd + d] = k_ref[e];
    kv.v[slot * kv.hd + d] = v_ref[e];
    if (d == 0) {
        kv.ks[slot] = ks_ref[(size_t)p * kv.nkv + h];
        kv.vs[slot] = vs_ref[(size_t)p * kv.nkv + h];
    }
}

__global__ void kv_export_kernel(int8_t* __restrict__ k_ref, float* __restrict__ ks_ref, int8_t* __restrict__ v_ref,
                                 float* __restrict__ vs_ref, int pos0, int npos, KVDev kv, int layer) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per = (size_t)kv.nkv * kv.hd;
    if (e >= (size_t)npos * per) return;
    const int p = (int)(e / per), rem = (int)(e % per), h = rem / kv.hd, d = rem % kv.hd;
    const size_t slot = ((size_t)layer * kv.nkv + h) * kv.max_seq + pos0 + p;
    k_ref[e] = kv.k[slot * kv.hd + d];
    v_ref[e] = kv.v[slot * kv.hd + d];
    if (d == 0) {
        ks_ref[(size_t)p * kv.nkv + h] = kv.ks[slot];
        vs_ref[(size_t)p * kv.nkv + h] = kv.vs[slot];
    }
}

void launch_kv_import(const int8_t* k_ref, const float* ks_ref, const int8_t* v_ref, const float* vs_ref, int pos0,
                      int npos, const KVDev& kv, int layer, hipStream_t st) {
    const size_t n = (size_t)npos * kv.nkv * kv.hd;
    hipLaunchKernelGGL(kv_import_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, k_ref, ks_ref, v_ref,
                       vs_ref, pos0, npos, kv, layer);
}

void launch_kv_export(int8_t* k_ref, float* ks_ref, int8_t* v_ref, float* vs_ref, int pos0, int npos,
                      const KVDev& kv, int layer, hipStream_t st) {
    const size_t n = (size_t)npos * kv.nkv * kv.hd;
    hipLaunchKernelGGL(kv_export_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, k_ref, ks_ref, v_ref,
                       vs_ref, pos0, npos, kv, layer);
}

// ---------------------------------------------------------------- clearing device memory

// n16 16-byte words of zeros, grid-strided (a kernel, so a captured graph holds no memset node)
__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* __restrict__ p, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

void launch_zero_fill(void* p, size_t bytes, hipStream_t st) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return;
    const unsigned grid = (unsigned)std::min<size_t>((n16 + 255) / 256, 2048);
    hipLaunchKernelGGL(zero_fill_kernel, dim3(grid), dim3(256), 0, st, reinterpret_cast<uint4*>(p), n16);
}

}  // namespace jy
