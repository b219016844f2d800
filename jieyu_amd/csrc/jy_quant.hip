// jy_quant.hip — weights of every type jieyu binds besides the Q8_0 fast path:
// k-quant (Q4_K / Q5_K / Q6_K) matrices in HBM, their decode matvec, and the
// per-type dispatch of matvec / GEMM that models of mixed weight types run.
//
// Decode matvec of a k-quant row = dot_row_avx2 (libs/matmul_libs/matmul_q.h:111-132):
// 32 virtual FMA lanes, lane L accumulates x[k] * w[k] for k = L mod 32 ascending,
// each 256-weight block dequantized as dequant_block does (:47-100), then the fixed
// tree s[i] = (a[i]+a[8+i]) + (a[16+i]+a[24+i]), r[i] = s[i]+s[4+i],
// y = (r0+r1)+(r2+r3).  The thread layout is the Q8_0 kernel's: 16 threads per row
// (two lanes each), 4 rows per wave, the activation vector lane-pair major in LDS.
#include <algorithm>

#include "jy_layout.h"

namespace jy {

// ---------------------------------------------------------------- layout

KQDev kq_shape(int type, int rows, int cols) {
    KQDev w;
    w.type = type;
    w.rows = rows;
    w.cols = cols;
    w.nsb = cols / 256;
    w.groups = (rows + 3) / 4;
    return w;
}

size_t kq_bytes(const KQDev& w, int part) {
    const size_t chunks = (size_t)w.groups * w.nsb;
    switch (part) {
        case 0: return chunks * 512;
        case 1: return w.type == JY_Q5_K ? chunks * 128 : w.type == JY_Q6_K ? chunks * 256 : 0;
        case 2: return chunks * 64;
        default: return chunks * 16;
    }
}

__host__ __device__ static inline int kq_block_bytes(int type) { return type == JY_Q4_K ? 144 : type == JY_Q5_K ? 176 : 210; }

// get_scale_min_k4 (libs/matmul_libs/matmul_q.h:22-33): the 6-bit scale and min of
// 32-weight step j of a Q4_K / Q5_K super-block
__device__ __forceinline__ void kq_scale_min(int j, const uint8_t* q, int& sc, int& mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// one thread per (row, super-block): GGML block -> the thread-major pieces.  Weight
// 32c + L (L = 2g + u) of the block goes to thread (row & 3) * 16 + g as weight (c, u).
__global__ void repack_kq_kernel(const uint8_t* __restrict__ src, KQDev W) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)W.rows * W.nsb) return;
    const int R = (int)(id / W.nsb), sb = (int)(id % W.nsb), ri = R & 3;
    const uint8_t* b = src + id * kq_block_bytes(W.type);
    const size_t chunk = (size_t)(R >> 2) * W.nsb + sb;
    for (int g = 0; g < 16; g++) {
        uint64_t nib = 0;
        uint32_t hb = 0;
        for (int c = 0; c < 8; c++)
            for (int u = 0; u < 2; u++) {
                const int L = 2 * g + u, T = 2 * (c >> 2) + u, kb = c & 3;
                uint32_t lo;
                if (W.type == JY_Q6_K) {  // matmul_q.h:78-96
                    const int nn = c >> 2, tq = c & 3;
                    const uint8_t qb = b[nn * 64 + L + 32 * (tq & 1)];
                    lo = tq < 2 ? (qb & 15u) : (qb >> 4);
                    hb |= ((b[128 + nn * 32 + L] >> (2 * tq)) & 3u) << (8 * kb + 2 * T);
                } else {  // q4.h:23-33, matmul_q.h:52-76
                    const uint8_t* qs = b + (W.type == JY_Q4_K ? 16 : 48);
                    const uint8_t qb = qs[(c >> 1) * 32 + L];
                    lo = (c & 1) ? (qb >> 4) : (qb & 15u);
                    if (W.type == JY_Q5_K) hb |= ((b[16 + L] >> c) & 1u) << (4 * T + kb);
                }
                nib |= (uint64_t)lo << (4 * (2 * c + u));
            }
        const size_t t = chunk * 64 + ri * 16 + g;
        *reinterpret_cast<uint64_t*>(W.nib + t * 8) = nib;
        if (W.type == JY_Q5_K) *reinterpret_cast<uint16_t*>(W.hi + t * 2) = (uint16_t)hb;
        if (W.type == JY_Q6_K) *reinterpret_cast<uint32_t*>(W.hi + t * 4) = hb;
    }
    uint8_t* h = W.hdr + chunk * 64 + ri * 16;
    if (W.type == JY_Q6_K) {
        // scale of step c for weights L < 16 (bytes 0..7) and L >= 16 (bytes 8..15):
        // sc[(c >> 2) * 8 + L / 16 + 2 * (c & 3)] of the block (matmul_q.h:83-90)
        for (int half = 0; half < 2; half++)
            for (int c = 0; c < 8; c++) h[half * 8 + c] = b[192 + (c >> 2) * 8 + half + 2 * (c & 3)];
        W.dm[chunk * 4 + ri] = (uint32_t)(b[208] | (b[209] << 8));
    } else {
        for (int c = 0; c < 8; c++) {
            int sc, mn;
            kq_scale_min(c, b + 4, sc, mn);
            h[c] = (uint8_t)sc;
            h[8 + c] = (uint8_t)mn;
        }
        W.dm[chunk * 4 + ri] = (uint32_t)(b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24));
    }
}

void launch_repack_kq(const uint8_t* src, const KQDev& dst, hipStream_t st) {
    const size_t n = (size_t)dst.rows * dst.nsb;
    hipLaunchKernelGGL(repack_kq_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, dst);
}

// ---------------------------------------------------------------- decode matvec

// byte j (a compile-time constant after unrolling) of a word, as a float: v_cvt_f32_ubyte
__device__ __forceinline__ float ubyte_f(uint32_t w, int j) { return (float)((w >> (8 * j)) & 255u); }

// the 16 weights of this thread in one chunk, fed to its two FMA lanes in order.
// Target word T (= 2*(c >> 2) + u) holds weight (c, u) in byte c & 3 after the mask,
// with the Q5_K / Q6_K high bits merged in above the nibble.
template <int TYPE>
__device__ __forceinline__ void kq_chunk(const uint2& nb, uint32_t hb, const uint4& h, uint32_t dmw, int g,
                                         const float* xv, float& a0, float& a1) {
    uint32_t wt[4] = {nb.x & 0x0F0F0F0Fu, (nb.x >> 4) & 0x0F0F0F0Fu, nb.y & 0x0F0F0F0Fu, (nb.y >> 4) & 0x0F0F0F0Fu};
    const float d = half_to_float((uint16_t)(dmw & 0xffffu));
    if (TYPE == JY_Q6_K) {
        // bits 8k + 2T of hb -> bits 4, 5 of byte k of word T
#pragma unroll
        for (int T = 0; T < 4; T++) wt[T] |= (T < 2 ? hb << (4 - 2 * T) : hb >> (2 * T - 4)) & 0x30303030u;
        const uint32_t s0 = g < 8 ? h.x : h.z, s1 = g < 8 ? h.y : h.w;  // the scales of this lane's half
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int8_t sc = (int8_t)((c < 4 ? s0 : s1) >> (8 * (c & 3)));
            const float ds = d * (float)sc;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                // (d*sc) * (q - 32), the reference's expression; q - 32 is exact
                const float w = ds * (ubyte_f(wt[2 * (c >> 2) + u], c & 3) - 32.0f);
                if (u == 0)
                    a0 = __builtin_fmaf(xv[2 * c], w, a0);
                else
                    a1 = __builtin_fmaf(xv[2 * c + 1], w, a1);
            }
        }
    } else {
        if (TYPE == JY_Q5_K) {
            // bit 4T + k of hb -> bit 4 of byte k of word T: spread the nibble by a multiply
#pragma unroll
            for (int T = 0; T < 4; T++) wt[T] |= ((((hb >> (4 * T)) & 15u) * 0x00204081u) << 4) & 0x10101010u;
        }
        const float dmin = half_to_float((uint16_t)(dmw >> 16));
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float d1 = d * ubyte_f(c < 4 ? h.x : h.y, c & 3), n1 = dmin * ubyte_f(c < 4 ? h.z : h.w, c & 3);
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float w = __builtin_fmaf(ubyte_f(wt[2 * (c >> 2) + u], c & 3), d1, -n1);
                if (u == 0)
                    a0 = __builtin_fmaf(xv[2 * c], w, a0);
                else
                    a1 = __builtin_fmaf(xv[2 * c + 1], w, a1);
            }
        }
    }
}

static constexpr int KQ_U = 4;  // chunks per register buffer (two buffers)

// one row group per wave, 4 waves per workgroup
template <int TYPE, int EPI>
__global__ __launch_bounds__(256) void matvec_kq_kernel(KQDev W, const float* __restrict__ x, float* __restrict__ out,
                                                        const float* __restrict__ aux) {
    extern __shared__ __align__(16) float xs[];  // [16][XS]: lane pair g, 16 floats per chunk
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane >> 4, g = lane & 15;
    const int K = W.cols, nsb = W.nsb, XS = 16 * nsb + 4;
    for (int k = tid; k < K; k += blockDim.x) xs[((k & 31) >> 1) * XS + 2 * (k >> 5) + (k & 1)] = x[k];
    __syncthreads();
    const int rg = blockIdx.x * 4 + wave;
    if (rg >= W.groups) return;
    const float* xrow = xs + g * XS;
    float a0 = 0.0f, a1 = 0.0f;
    const size_t c0 = (size_t)rg * nsb;
    // two buffers of KQ_U chunks: the next buffer's loads are in flight while the
    // current one is computed (chunk indices past the row clamp to its last chunk)
    struct Buf {
        uint2 nb[KQ_U];
        uint32_t hb[KQ_U];
        uint4 h[KQ_U];
        uint32_t dm[KQ_U];
    };
    auto load = [&](Buf& b, int s0) {
#pragma unroll
        for (int u = 0; u < KQ_U; u++) {
            const size_t c = c0 + min(s0 + u, nsb - 1);
            b.nb[u] = *reinterpret_cast<const uint2*>(W.nib + (c * 64 + lane) * 8);
            b.hb[u] = TYPE == JY_Q5_K   ? *reinterpret_cast<const uint16_t*>(W.hi + (c * 64 + lane) * 2)
                      : TYPE == JY_Q6_K ? *reinterpret_cast<const uint32_t*>(W.hi + (c * 64 + lane) * 4)
                                        : 0u;
            b.h[u] = *reinterpret_cast<const uint4*>(W.hdr + c * 64 + r * 16);
            b.dm[u] = W.dm[c * 4 + r];
        }
    };
    auto compute = [&](const Buf& b, int s0) {
#pragma unroll
        for (int u = 0; u < KQ_U; u++) {
            if (s0 + u < nsb) {
                float xv[16];
                const float4* xp = reinterpret_cast<const float4*>(xrow + 16 * (s0 + u));
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 v = xp[q];
                    xv[4 * q] = v.x;
                    xv[4 * q + 1] = v.y;
                    xv[4 * q + 2] = v.z;
                    xv[4 * q + 3] = v.w;
                }
                kq_chunk<TYPE>(b.nb[u], b.hb[u], b.h[u], b.dm[u], g, xv, a0, a1);
            }
        }
    };
    Buf A, B;
    load(A, 0);
    for (int s0 = 0; s0 < nsb; s0 += 2 * KQ_U) {
        load(B, s0 + KQ_U);
        compute(A, s0);
        if (s0 + 2 * KQ_U < nsb) load(A, s0 + 2 * KQ_U);
        compute(B, s0 + KQ_U);
    }
    // lanes 2g, 2g+1 -> the reference's reduction tree (as in the Q8_0 matvec)
    a0 += dpp_f<0x12C>(a0);
    a1 += dpp_f<0x12C>(a1);
    a0 += dpp_f<0x128>(a0);
    a1 += dpp_f<0x128>(a1);
    a0 += dpp_f<0x4E>(a0);
    a1 += dpp_f<0x4E>(a1);
    const float t = a0 + a1;
    const float y = t + dpp_f<0xB1>(t);
    const int row = rg * 4 + r;
    if (g == 0 && row < W.rows) {
        if (EPI == EPI_STORE) out[row] = y;
        if (EPI == EPI_BIAS) out[row] = y + aux[row];
        if (EPI == EPI_RESID) out[row] = out[row] + y;
    }
}

size_t mv_kq_lds_bytes(int cols) { return (size_t)16 * (16 * (cols / 256) + 4) * sizeof(float); }

template <int TYPE>
static void mv_kq(const KQDev& W, const float* x, float* out, Epi epi, const float* aux, hipStream_t st) {
    const dim3 grid((unsigned)((W.groups + 3) / 4)), block(256);
    const size_t lds = mv_kq_lds_bytes(W.cols);
    if (epi == EPI_STORE) hipLaunchKernelGGL((matvec_kq_kernel<TYPE, EPI_STORE>), grid, block, lds, st, W, x, out, aux);
    if (epi == EPI_BIAS) hipLaunchKernelGGL((matvec_kq_kernel<TYPE, EPI_BIAS>), grid, block, lds, st, W, x, out, aux);
    if (epi == EPI_RESID) hipLaunchKernelGGL((matvec_kq_kernel<TYPE, EPI_RESID>), grid, block, lds, st, W, x, out, aux);
}

void launch_mv(const DevW& W, const float* x, float* out, Epi epi, const float* aux, hipStream_t st) {
    switch (W.type) {
        case JY_F32:
            launch_matvec_f32(static_cast<const float*>(W.dense), W.in, W.out, x, out, aux, epi, st);
            break;
        case JY_F16: launch_matvec_f16(static_cast<const uint16_t*>(W.dense), W.in, W.out, x, out, aux, epi, st); break;
        case JY_Q8_0: {
            MvArgs a;
            a.aux = aux;
            launch_matvec_q8(W.q8, x, nullptr, out, epi, a, st);
            break;
        }
        case JY_Q4_K: mv_kq<JY_Q4_K>(W.kq, x, out, epi, aux, st); break;
        case JY_Q5_K: mv_kq<JY_Q5_K>(W.kq, x, out, epi, aux, st); break;
        case JY_Q6_K: mv_kq<JY_Q6_K>(W.kq, x, out, epi, aux, st); break;
        default: break;
    }
}

template <int TYPE>
static hipError_t kq_attr() {
    hipError_t e = hipSuccess;
    for (const void* f : {reinterpret_cast<const void*>(&matvec_kq_kernel<TYPE, EPI_STORE>),
                          reinterpret_cast<const void*>(&matvec_kq_kernel<TYPE, EPI_BIAS>),
                          reinterpret_cast<const void*>(&matvec_kq_kernel<TYPE, EPI_RESID>)})
        if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 2048);
    return e;
}

hipError_t quant_init() {
    for (hipError_t e : {kq_attr<JY_Q4_K>(), kq_attr<JY_Q5_K>(), kq_attr<JY_Q6_K>()})
        if (e != hipSuccess) return e;
    return hipSuccess;
}

}  // namespace jy
