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
// Tiling.  A workgroup of 2 x 2 waves computes 64 rows (tokens) x 64 NT columns (matrix
// rows), each wave 32 x 16 NT: 2 x NT tiles of 16 x 16, acc in the MFMA C layout (lane l
// holds rows 4 (l/16) .. +3 of column l % 16).  The operands reach LDS by global -> LDS DMA
// three blocks deep (activation parts in operand order, weights as stored, block scales),
// one workgroup barrier per block; each wave converts its weight fragments to fp16.
#include <algorithm>
#include <cstddef>

#include "jy_layout.h"
#include "jy_mfma.h"

namespace jy {

static constexpr int GM_TILE = 128;  // activation rows are padded to a multiple of this

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));

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

// one row of the padded activations (LDS or global, K values; `live` false: the row past m,
// zero) into its fp16 high / low parts and its unscale, by a workgroup of 256 threads
__device__ __forceinline__ void split_row(const float* a, bool live, int K, int row, _Float16* __restrict__ hi,
                                          _Float16* __restrict__ lo, float* __restrict__ unscale, float* red) {
    const int tid = threadIdx.x;
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

// one workgroup per row of the padded activations [mp][K]: rows past m are zero
__global__ __launch_bounds__(256) void mfma_split_kernel(const float* __restrict__ A, int m, int K,
                                                         _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                         float* __restrict__ unscale) {
    __shared__ float red[4];
    split_row(A + (size_t)blockIdx.x * K, (int)blockIdx.x < m, K, blockIdx.x, hi, lo, unscale, red);
}

// the same after the row's RMSNorm (block_rmsnorm, as rmsnorm_kernel computes it, in place in
// LDS): one kernel and one pass over the row instead of two
__global__ __launch_bounds__(256) void mfma_norm_split_kernel(const float* __restrict__ X, int m, int K,
                                                              const float* __restrict__ nw, _Float16* __restrict__ hi,
                                                              _Float16* __restrict__ lo,
                                                              float* __restrict__ unscale) {
    extern __shared__ __align__(16) float xr[];
    __shared__ float red[18];
    const bool live = (int)blockIdx.x < m;
    if (live) {
        const float* x = X + (size_t)blockIdx.x * K;
        for (int i = threadIdx.x; i < K; i += 256) xr[i] = x[i];
        __syncthreads();
        block_rmsnorm(xr, K, nw, xr, red);
        __syncthreads();
    }
    split_row(xr, live, K, blockIdx.x, hi, lo, unscale, red);
}

// The same two kernels with the row in registers: NV float4s per thread (element
// 4 (tid + 256 j) .. +3 in v[j]), one read of the row, 16-byte loads and 8-byte stores of
// four halves; the same arithmetic element by element (K a multiple of 4, K <= 1024 NV).
template <int NV>
__device__ __forceinline__ void split_row4(const float4 (&v)[NV], int K, int row, _Float16* __restrict__ hi,
                                           _Float16* __restrict__ lo, float* __restrict__ unscale, float* red) {
    const int tid = threadIdx.x;
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++)
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    amax = wave_max64(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int ex = 0;
    if (amax > 0.0f) frexpf(amax, &ex);
    const int s = amax > 0.0f ? min(max(14 - ex, -100), 100) : 0;
    const float up = ldexpf(1.0f, s);
    if (tid == 0) unscale[row] = ldexpf(1.0f, -s);
    _Float16* h = hi + (size_t)row * K;
    _Float16* w = lo + (size_t)row * K;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k4 = tid + 256 * j;
        if (4 * k4 >= K) break;
        const float e[4] = {v[j].x * up, v[j].y * up, v[j].z * up, v[j].w * up};
        h4_t vh, vl;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            vh[i] = (_Float16)e[i];
            vl[i] = (_Float16)(e[i] - (float)vh[i]);
        }
        *reinterpret_cast<h4_t*>(h + 4 * k4) = vh;
        *reinterpret_cast<h4_t*>(w + 4 * k4) = vl;
    }
}

template <int NV>
__global__ __launch_bounds__(256) void mfma_split4_kernel(const float* __restrict__ A, int m, int K,
                                                          _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                          float* __restrict__ unscale) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const bool live = row < m;
    const float4* a4 = reinterpret_cast<const float4*>(A + (size_t)row * K);
    float4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k4 = threadIdx.x + 256 * j;
        v[j] = live && 4 * k4 < K ? a4[k4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    split_row4<NV>(v, K, row, hi, lo, unscale, red);
}

// (kz > 1: X's rows first take the residual add of a GEMM split over K whose sum was
// deferred, X += sum of the kz partials [kz][m][K] in slice order, written back to X: the
// sum kernel's arithmetic)
template <int NV>
__global__ __launch_bounds__(256) void mfma_norm_split4_kernel(float* __restrict__ X, int m, int K,
                                                               const float* __restrict__ nw, _Float16* __restrict__ hi,
                                                               _Float16* __restrict__ lo, float* __restrict__ unscale,
                                                               const float* __restrict__ kp, int kz) {
    extern __shared__ __align__(16) float xr[];
    __shared__ float red[18];
    const int row = blockIdx.x;
    const bool live = row < m;
    float4* x4 = reinterpret_cast<float4*>(xr);
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // the norm weights go out first (they do not wait for the row), the row to registers
    // and to LDS for the sum of squares in the reference's lane order
    float4 w4[NV], v[NV];
    const float4* n4 = reinterpret_cast<const float4*>(nw);
    const float4* g4 = reinterpret_cast<const float4*>(X + (size_t)row * K);
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k4 = threadIdx.x + 256 * j;
        w4[j] = live && 4 * k4 < K ? n4[k4] : z4;
        v[j] = live && 4 * k4 < K ? g4[k4] : z4;
    }
    if (kz > 1 && live) {
        const size_t mk4 = (size_t)m * K / 4;
        const float4* p4 = reinterpret_cast<const float4*>(kp) + (size_t)row * K / 4;
        float4* xw4 = reinterpret_cast<float4*>(X + (size_t)row * K);
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int k4 = threadIdx.x + 256 * j;
            if (4 * k4 >= K) break;
            float4 y = p4[k4];
            for (int z = 1; z < kz; z++) {
                const float4 t = p4[(size_t)z * mk4 + k4];
                y = make_float4(y.x + t.x, y.y + t.y, y.z + t.z, y.w + t.w);
            }
            v[j] = make_float4(v[j].x + y.x, v[j].y + y.y, v[j].z + y.z, v[j].w + y.w);
            xw4[k4] = v[j];
        }
    }
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k4 = threadIdx.x + 256 * j;
        if (live && 4 * k4 < K) x4[k4] = v[j];
    }
    if (live) {
        __syncthreads();
        block_rms_scale(xr, K, red);
        // y = (x * scale) * w, as block_rmsnorm computes it
        const float scale = red[16];
        const bool zero = red[17] != 0.0f;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            v[j].x = zero ? 0.0f : (v[j].x * scale) * w4[j].x;
            v[j].y = zero ? 0.0f : (v[j].y * scale) * w4[j].y;
            v[j].z = zero ? 0.0f : (v[j].z * scale) * w4[j].z;
            v[j].w = zero ? 0.0f : (v[j].w * scale) * w4[j].w;
        }
        __syncthreads();  // (red is reused below)
    }
    split_row4<NV>(v, K, row, hi, lo, unscale, red);
}

// float4s per thread for a row of K (0: the scalar kernels: K not a multiple of 4 or past 16384)
static int split_nv(int K) {
    if (K % 4 || K > 16384) return 0;
    const int n = (K + 1023) / 1024;
    return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : n <= 8 ? 8 : 16;
}

bool mfma_norm_split_takes_parts(int K) { return split_nv(K) != 0; }

void launch_mfma_norm_split(float* X, int m, int mp, int K, const float* nw, _Float16* hi, _Float16* lo,
                            float* unscale, hipStream_t st, const float* kp, int kz) {
    const size_t lds = (size_t)K * sizeof(float);
    switch (split_nv(K)) {
        case 1: hipLaunchKernelGGL(mfma_norm_split4_kernel<1>, dim3(mp), dim3(256), lds, st, X, m, K, nw, hi, lo, unscale, kp, kz); break;
        case 2: hipLaunchKernelGGL(mfma_norm_split4_kernel<2>, dim3(mp), dim3(256), lds, st, X, m, K, nw, hi, lo, unscale, kp, kz); break;
        case 4: hipLaunchKernelGGL(mfma_norm_split4_kernel<4>, dim3(mp), dim3(256), lds, st, X, m, K, nw, hi, lo, unscale, kp, kz); break;
        case 8: hipLaunchKernelGGL(mfma_norm_split4_kernel<8>, dim3(mp), dim3(256), lds, st, X, m, K, nw, hi, lo, unscale, kp, kz); break;
        case 16: hipLaunchKernelGGL(mfma_norm_split4_kernel<16>, dim3(mp), dim3(256), lds, st, X, m, K, nw, hi, lo, unscale, kp, kz); break;
        default:  // (callers pass no partials here: mfma_norm_split_takes_parts)
            hipLaunchKernelGGL(mfma_norm_split_kernel, dim3(mp), dim3(256), lds, st, X, m, K, nw, hi, lo, unscale);
            break;
    }
}

void launch_mfma_split(const float* A, int m, int mp, int K, _Float16* hi, _Float16* lo, float* unscale,
                       hipStream_t st) {
    switch (split_nv(K)) {
        case 1: hipLaunchKernelGGL(mfma_split4_kernel<1>, dim3(mp), dim3(256), 0, st, A, m, K, hi, lo, unscale); break;
        case 2: hipLaunchKernelGGL(mfma_split4_kernel<2>, dim3(mp), dim3(256), 0, st, A, m, K, hi, lo, unscale); break;
        case 4: hipLaunchKernelGGL(mfma_split4_kernel<4>, dim3(mp), dim3(256), 0, st, A, m, K, hi, lo, unscale); break;
        case 8: hipLaunchKernelGGL(mfma_split4_kernel<8>, dim3(mp), dim3(256), 0, st, A, m, K, hi, lo, unscale); break;
        case 16: hipLaunchKernelGGL(mfma_split4_kernel<16>, dim3(mp), dim3(256), 0, st, A, m, K, hi, lo, unscale); break;
        default: hipLaunchKernelGGL(mfma_split_kernel, dim3(mp), dim3(256), 0, st, A, m, K, hi, lo, unscale); break;
    }
}

// ---------------------------------------------------------------- the GEMM, staged by DMA
//
// Per block: the hi-part MFMA, the lo-part MFMA into the same sum, one fp32 fma with the
// block scale.  The operands are brought to LDS by global -> LDS DMA, S blocks deep, with
// a wave tile of
// 16 MT token rows x 16 NT columns (a workgroup of 2 x 2 waves: 32 MT x 32 NT).  The
// weights stay int8 in LDS (8 bytes per lane per 16 x 32 tile) and become fp16 per
// fragment (q8_to_h8).  Per block a wave reads 2 MT KiB of activation fragments and NT / 2
// KiB of weights from LDS for 2 MT NT matrix operations.  (A register-staged form with one
// 32-weight block per barrier, 64 x 64 per wave and the weight fragments read twice was
// bound by LDS reads: gate/up at 1024 tokens 682 us against 576 here.)

// global -> LDS DMA (16 or 4 bytes per lane: lane l writes at the M0 base + l * size),
// issued as inline assembly: the compiler cannot tell a DMA's LDS destination from the LDS
// the waves read and would wait for every DMA before each LDS access; the kernel instead
// waits for its own DMAs explicitly before the barrier that publishes a stage.  The asm sets
// M0 itself; nothing else in these kernels uses M0 (checked in the generated code).
// (M0 is a reserved register: the compiler warns that naming it as clobbered may not be
// honoured, which is harmless here since no compiler-generated code in these kernels uses it)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_b128(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma_b32(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ uint32_t lds_byte_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char*)p;
}

// s_waitcnt with only vmcnt <= n (n < 64)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// one stage: activation fragments [part][row tile][lane], weights [column tile][lane]
// (8 bytes: lanes 0..31 of a 16-byte DMA cover one tile), block scales [column tile][row]
template <int MT, int NT>
struct G2Stage {
    h8_t a[2][2 * MT][64];
    uint2 b[2 * NT][64];
    float d[2 * NT][16];
};

template <int EPI, int MT, int NT, int S>
__global__ __launch_bounds__(256, 2) void gemm_q8_mfma2_kernel(Q8MfmaDev W, int m, int K, const _Float16* __restrict__ ahi,
                                                            const _Float16* __restrict__ alo,
                                                            const float* __restrict__ unscale, float* __restrict__ C,
                                                            int ldc, const float* __restrict__ aux) {
    static_assert(MT == 2 || MT == 4, "row tiles per wave");
    static_assert(NT == 4 || NT == 8, "column tiles per wave");
    static_assert(S == 3 || S == 4, "stages");
    using St = G2Stage<MT, NT>;
    extern __shared__ __align__(16) unsigned char g2smem[];
    St* stg = reinterpret_cast<St*>(g2smem);
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int c = l & 15, G = l >> 4;
    const int rowt = blockIdx.x * 32 * MT;  // the workgroup's first token row
    const int tilet = blockIdx.y * 2 * NT;  // its first 16-column tile
    const int nb = W.nb;
    // the workgroup's K slice: blocks [b0, b1) of gridDim.z slices of nbz (all of them with
    // one slice), its sums into C's slice z ([z][m][ldc]: the partials a sum kernel adds)
    const int nbz = (nb + (int)gridDim.z - 1) / (int)gridDim.z;
    const int b0 = (int)blockIdx.z * nbz, b1 = min(nb, b0 + nbz);
    C += (size_t)blockIdx.z * m * ldc;
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_byte_addr(g2smem));
    constexpr int PW = MT + NT / 4 + 1;  // DMA instructions per wave per block

    // block b into stage s: this wave's share of the 4 MT activation, NT weight and 4 scale
    // DMA instructions (the same count for every wave)
    auto issue = [&](int b, int s) {
        const uint32_t sb = base + (uint32_t)(s * sizeof(St));
#pragma unroll
        for (int j = 0; j < MT; j++) {
            const int i = wave * MT + j, part = i / (2 * MT), rt = i % (2 * MT);
            const _Float16* src = (part ? alo : ahi) + (size_t)(rowt + 16 * rt + c) * K + 32 * b + 8 * G;
            dma_b128(src, sb + (uint32_t)(offsetof(St, a) + (size_t)(part * 2 * MT + rt) * 64 * 16));
        }
#pragma unroll
        for (int j = 0; j < NT / 4; j++) {
            const int jj = wave * (NT / 4) + j, t = 2 * jj + (l >> 5);
            const int tg = min(tilet + t, W.tiles - 1);
            const int8_t* src = W.q + ((size_t)tg * nb + b) * 512 + (l & 31) * 16;
            dma_b128(src, sb + (uint32_t)(offsetof(St, b) + (size_t)(2 * jj) * 512));
        }
        {
            const int f = wave * 8 * NT + l, t = f >> 4, r = f & 15;
            const int tg = min(tilet + t, W.tiles - 1);
            const float* src = W.d + ((size_t)(tg * W.nb4 + (b >> 2)) * 16 + r) * 4 + (b & 3);
            if (l < 8 * NT) dma_b32(src, sb + (uint32_t)(offsetof(St, d) + (size_t)wave * 8 * NT * 4));
        }
    };

    f4_t acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // The narrow tile (NT = 4) runs the block loop software-pipelined; the wide tile's
    // registers do not hold a second set of fragments well (238 VGPRs: gate/up 594 -> 628 us),
    // so it reads each block's fragments after its barrier.
    if constexpr (NT == 4) {
        // Software-pipelined over blocks: while the matrix cores work on block b from registers,
        // the fragments of block b + 1 are read from LDS into the other register set.  S blocks
        // are in LDS or in flight: block b + S goes into block b's stage once every wave has
        // read block b (the barrier before block b + 1's reads).
        struct Frag {
            h8_t ah[MT], al[MT];
            uint2 q[NT];
            float dj[NT];
        };
        auto read_frag = [&](int b, Frag& f) {
            const St& T = stg[(b - b0) % S];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                f.ah[mt] = T.a[0][wm * MT + mt][l];
                f.al[mt] = T.a[1][wm * MT + mt][l];
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                f.q[nt] = T.b[wn * NT + nt][l];
                f.dj[nt] = T.d[wn * NT + nt][c];
            }
        };
        // the wait for block b's DMAs when `later` blocks were issued after it
        auto wait_block = [&](int later) {
            if (later >= S - 1)
                wait_vm<(S - 1) * PW>();
            else if (later == S - 2)
                wait_vm<(S - 2) * PW>();
            else if (S > 3 && later == 1)
                wait_vm<(S > 3 ? PW : 0)>();
            else
                wait_vm<0>();
        };
        auto compute = [&](const Frag& f) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const h8_t bq = q8_to_h8(f.q[nt].x, f.q[nt].y);
                f4_t t[MT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.ah[mt], bq, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.al[mt], bq, t[mt], 0, 0, 0);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[mt][nt][i] = __builtin_fmaf(f.dj[nt], t[mt][i], acc[mt][nt][i]);
            }
        };
        // block b from cur; block b + 1 (if any) into nxt
        auto step = [&](int b, const Frag& cur, Frag& nxt) {
            if (b + 1 < b1) {
                // issued after block b + 1 so far: blocks b + 2 .. min(b + S - 1, b1 - 1)
                wait_block(min(S - 2, b1 - b - 2));
                __syncthreads();  // block b + 1 is in LDS; every wave has read block b
                if (b + S < b1) issue(b + S, (b - b0) % S);
                read_frag(b + 1, nxt);
            }
            compute(cur);
        };

#pragma unroll
        for (int s = 0; s < S; s++)
            if (b0 + s < b1) issue(b0 + s, s);
        Frag fa, fb;
        if (b0 < b1) {
            wait_block(min(S - 1, b1 - b0 - 1));
            __syncthreads();
            read_frag(b0, fa);
        }
        int b = b0;
        for (; b + 1 < b1; b += 2) {
            step(b, fa, fb);
            step(b + 1, fb, fa);
        }
        if (b < b1) step(b, fa, fb);
    } else {
#pragma unroll
        for (int s = 0; s < S - 1; s++)
            if (b0 + s < b1) issue(b0 + s, s);
        for (int b = b0; b < b1; b++) {
            // block b has landed once at most the DMAs of the S - 2 blocks after it are pending
            const int after = min(b1 - 1 - b, S - 2);
            if (after >= S - 2)
                wait_vm<(S - 2) * PW>();
            else if (S > 3 && after == 1)
                wait_vm<(S > 3 ? PW : 0)>();
            else
                wait_vm<0>();
            __syncthreads();  // every wave's DMAs of block b are in LDS; block b - 1 is done
            if (b + S - 1 < b1) issue(b + S - 1, (b - b0 + S - 1) % S);
            const St& T = stg[(b - b0) % S];
            h8_t ah[MT], al[MT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                ah[mt] = T.a[0][wm * MT + mt][l];
                al[mt] = T.a[1][wm * MT + mt][l];
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const uint2 q = T.b[wn * NT + nt][l];
                const h8_t bq = q8_to_h8(q.x, q.y);
                const float dj = T.d[wn * NT + nt][c];
                f4_t t[MT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt], bq, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt], bq, t[mt], 0, 0, 0);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[mt][nt][i] = __builtin_fmaf(dj, t[mt][i], acc[mt][nt][i]);
            }
        }
    }

    // epilogue: acc[mt][nt][i] is C[row][col] before the row's unscale; the rows' factors
    // are loaded together first, so no store waits for a load of its own
    const int N = W.rows;
    float us[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = rowt + wm * 16 * MT + 16 * mt + 4 * G + i;
            us[mt][i] = row < m ? unscale[row] : 0.0f;
        }
    if (EPI == EPI_SWIGLU) {
        // the gate/up matrix's rows 2j, 2j+1 are gate_j, up_j: columns 2j and 2j+1 of C lie in
        // lanes c and c + 1 of a tile; the even lane writes h[row][j] = silu(gate) * up with
        // the reference's SiLU of element row * F + j of the m x F array (silu_mul_kernel)
        const int F = N >> 1;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            if (tilet + wn * NT + nt >= W.tiles) continue;  // (uniform over the wave)
            const int col = 16 * (tilet + wn * NT + nt) + c;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int row = rowt + wm * 16 * MT + 16 * mt + 4 * G + i;
                    const float y = acc[mt][nt][i] * us[mt][i];
                    const float up = __shfl_xor(y, 1);
                    if (!(c & 1) && col + 1 < N && row < m) {
                        const int j = col >> 1;
                        C[(size_t)row * ldc + j] = silu_at(y, (size_t)row * F + j, (size_t)m * F) * up;
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int col = 16 * (tilet + wn * NT + nt) + c;
        if (tilet + wn * NT + nt >= W.tiles || col >= N) continue;
        const float bias = EPI == EPI_BIAS ? aux[col] : 0.0f;
        float old[MT][4];
        if (EPI == EPI_RESID) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int row = rowt + wm * 16 * MT + 16 * mt + 4 * G + i;
                    old[mt][i] = row < m ? C[(size_t)row * ldc + col] : 0.0f;
                }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = rowt + wm * 16 * MT + 16 * mt + 4 * G + i;
                if (row >= m) continue;
                const float y = acc[mt][nt][i] * us[mt][i];
                C[(size_t)row * ldc + col] = EPI == EPI_RESID ? old[mt][i] + y : y + bias;
            }
    }
}

int mfma_rows_padded(int m) { return (m + GM_TILE - 1) / GM_TILE * GM_TILE; }

// ---------------------------------------------------------------- split over K
//
// A grid of fewer workgroups than CUs (the small matrices of a short prompt) leaves most of
// the chip idle and each wave walking a long chain of blocks alone.  Such a GEMM runs as Z
// slices of K (gridDim.z), each writing its partial sums [z][m][N] (plain stores), then
// gemm_ksum_kernel adds the partials in slice order and applies the epilogue: the same
// result for every run, whatever order the slices finish in.

static constexpr int KSPLIT_MAX = 8;         // slices
static constexpr int KSPLIT_MIN_BLOCKS = 8;  // 32-weight blocks per slice, at least

template <int EPI>
__global__ __launch_bounds__(256) void gemm_ksum_kernel(const float* __restrict__ P, int Z, int m, int N,
                                                        float* __restrict__ C, int ldc, const float* __restrict__ aux) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t mn = (size_t)m * N;
    if (i >= mn) return;
    const int row = (int)(i / N), col = (int)(i - (size_t)row * N);
    float v[KSPLIT_MAX];
#pragma unroll
    for (int z = 0; z < KSPLIT_MAX; z++) v[z] = z < Z ? P[(size_t)z * mn + i] : 0.0f;
    float y = v[0];
#pragma unroll
    for (int z = 1; z < KSPLIT_MAX; z++)
        if (z < Z) y += v[z];
    float* c = C + (size_t)row * ldc + col;
    if (EPI == EPI_RESID)
        *c = *c + y;
    else if (EPI == EPI_BIAS)
        *c = y + aux[col];
    else
        *c = y;
}

template <int MT, int NT, int S>
static size_t g2_lds() {
    return (size_t)S * sizeof(G2Stage<MT, NT>);
}

template <int MT, int NT, int S>
static void gemm2_launch(const Q8MfmaDev& W, int m, const _Float16* hi, const _Float16* lo, const float* unscale,
                         float* C, int ldc, const float* aux, Epi epi, hipStream_t st, int Z = 1) {
    const dim3 grid((unsigned)(mfma_rows_padded(m) / (32 * MT)), (unsigned)((W.tiles + 2 * NT - 1) / (2 * NT)),
                    (unsigned)Z);
    const int K = W.nb * 32;
    const size_t lds = g2_lds<MT, NT, S>();
    switch (epi) {
        case EPI_BIAS:
            hipLaunchKernelGGL((gemm_q8_mfma2_kernel<EPI_BIAS, MT, NT, S>), grid, dim3(256), lds, st, W, m, K, hi, lo,
                               unscale, C, ldc, aux);
            break;
        case EPI_RESID:
            hipLaunchKernelGGL((gemm_q8_mfma2_kernel<EPI_RESID, MT, NT, S>), grid, dim3(256), lds, st, W, m, K, hi, lo,
                               unscale, C, ldc, aux);
            break;
        case EPI_SWIGLU:
            hipLaunchKernelGGL((gemm_q8_mfma2_kernel<EPI_SWIGLU, MT, NT, S>), grid, dim3(256), lds, st, W, m, K, hi, lo,
                               unscale, C, ldc, aux);
            break;
        default:
            hipLaunchKernelGGL((gemm_q8_mfma2_kernel<EPI_STORE, MT, NT, S>), grid, dim3(256), lds, st, W, m, K, hi, lo,
                               unscale, C, ldc, aux);
            break;
    }
}

template <int MT, int NT, int S>
static hipError_t gemm2_attr() {
    hipError_t e = hipSuccess;
    for (const void* f : {reinterpret_cast<const void*>(&gemm_q8_mfma2_kernel<EPI_STORE, MT, NT, S>),
                          reinterpret_cast<const void*>(&gemm_q8_mfma2_kernel<EPI_BIAS, MT, NT, S>),
                          reinterpret_cast<const void*>(&gemm_q8_mfma2_kernel<EPI_RESID, MT, NT, S>),
                          reinterpret_cast<const void*>(&gemm_q8_mfma2_kernel<EPI_SWIGLU, MT, NT, S>)})
        if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)g2_lds<MT, NT, S>());
    return e;
}

hipError_t gemm_mfma_init() {
    hipError_t e = gemm2_attr<2, 8, 3>();
    if (e == hipSuccess) e = gemm2_attr<2, 4, 3>();
    return e;
}

static int g_gemm_cus = 0;

static int gemm_cus() {
    if (!g_gemm_cus) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            g_gemm_cus = cus;
        else
            g_gemm_cus = 256;
    }
    return g_gemm_cus;
}

// workgroups of the wide tile's grid (128 columns per wave)
static long wide_wgs(const Q8MfmaDev& W, int m) { return (long)(mfma_rows_padded(m) / 64) * ((W.tiles + 15) / 16); }

// K slices for C = A W^T over m rows: 1 unless the narrow tile's grid has fewer workgroups
// than CUs; then up to two workgroups per CU, at most KSPLIT_MAX slices of at least
// KSPLIT_MIN_BLOCKS blocks, none of them empty.  (The SwiGLU epilogue pairs columns and is
// not split.)
int gemm_q8_mfma_ksplit(const Q8MfmaDev& W, int m, Epi epi) {
    const int cus = gemm_cus();
    const long wgs = (long)(mfma_rows_padded(m) / 64) * ((W.tiles + 7) / 8);
    if (epi == EPI_SWIGLU || wide_wgs(W, m) >= 2L * cus || wgs >= cus) return 1;
    const int z = (int)std::min<long>(std::min<long>(KSPLIT_MAX, 2L * cus / std::max(1L, wgs)),
                                      W.nb / KSPLIT_MIN_BLOCKS);
    if (z < 2) return 1;
    const int nbz = (W.nb + z - 1) / z;
    return (W.nb + nbz - 1) / nbz;
}

size_t gemm_q8_mfma_kpart_floats(const Q8MfmaDev& W, int m, Epi epi) {
    const int z = gemm_q8_mfma_ksplit(W, m, epi);
    return z > 1 ? (size_t)z * m * W.rows : 0;
}

// the wide tile (128 columns per wave) when its grid gives every CU at least two
// workgroups, else the narrow one (64 columns per wave, twice the workgroups), split over K
// when even that grid leaves CUs idle and `kpart` holds the partials.  Measured at the
// Llama-3-8B shapes and 1024 tokens (the activation split included): gate/up (28672 x
// 4096) 576 us wide, 686 narrow; QKV 164, O 118, down 422 us narrow.
int launch_gemm_q8_mfma(const Q8MfmaDev& W, int m, const _Float16* hi, const _Float16* lo, const float* unscale,
                        float* C, int ldc, const float* aux, Epi epi, hipStream_t st, float* kpart, size_t kpart_n,
                        bool defer) {
    const int cus = gemm_cus();
    if (wide_wgs(W, m) >= 2L * cus) {
        gemm2_launch<2, 8, 3>(W, m, hi, lo, unscale, C, ldc, aux, epi, st);
        return 0;
    }
    const int Z = gemm_q8_mfma_ksplit(W, m, epi);
    if (Z < 2 || !kpart || (size_t)Z * m * W.rows > kpart_n) {
        gemm2_launch<2, 4, 3>(W, m, hi, lo, unscale, C, ldc, aux, epi, st);
        return 0;
    }
    gemm2_launch<2, 4, 3>(W, m, hi, lo, unscale, kpart, W.rows, nullptr, EPI_STORE, st, Z);
    if (defer) return Z;
    const size_t n = (size_t)m * W.rows;
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (epi) {
        case EPI_BIAS:
            hipLaunchKernelGGL(gemm_ksum_kernel<EPI_BIAS>, grid, dim3(256), 0, st, kpart, Z, m, W.rows, C, ldc, aux);
            break;
        case EPI_RESID:
            hipLaunchKernelGGL(gemm_ksum_kernel<EPI_RESID>, grid, dim3(256), 0, st, kpart, Z, m, W.rows, C, ldc, aux);
            break;
        default:
            hipLaunchKernelGGL(gemm_ksum_kernel<EPI_STORE>, grid, dim3(256), 0, st, kpart, Z, m, W.rows, C, ldc, aux);
            break;
    }
    return 0;
}

void launch_gemm_ksum(const float* kpart, int Z, int m, int N, float* C, int ldc, const float* aux, Epi epi,
                      hipStream_t st) {
    const dim3 grid((unsigned)(((size_t)m * N + 255) / 256));
    if (epi == EPI_RESID)
        hipLaunchKernelGGL(gemm_ksum_kernel<EPI_RESID>, grid, dim3(256), 0, st, kpart, Z, m, N, C, ldc, aux);
    else if (epi == EPI_BIAS)
        hipLaunchKernelGGL(gemm_ksum_kernel<EPI_BIAS>, grid, dim3(256), 0, st, kpart, Z, m, N, C, ldc, aux);
    else
        hipLaunchKernelGGL(gemm_ksum_kernel<EPI_STORE>, grid, dim3(256), 0, st, kpart, Z, m, N, C, ldc, aux);
}

}  // namespace jy
