// jy_device.h — device-side arithmetic shared by the decode kernels.
//
// Each helper reproduces one piece of jieyu's CPU arithmetic bit for bit.  The
// kernels are compiled with -ffp-contract=off, so only the explicit
// __builtin_fmaf / __builtin_fma calls fuse; float division and sqrtf are the
// correctly rounded IEEE operations (hipcc's default), like SSE's divss/sqrtss.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jy {

// IEEE half -> float.  Every half, subnormals included, is exact in float, which
// is the value libs/date_libs/wmat.h:8-24 builds bit by bit.
__host__ __device__ __forceinline__ float half_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// expf with the results of the host libm the reference links (glibc 2.35,
// x86-64 FMA variant): the published exp2f-table algorithm of ARM's
// optimized-routines (32-entry table, cubic in double), with the contractions
// GCC forms when that C is built with FMA.  Checked bit-exact against glibc's
// expf on all 2^32 inputs on the host; the softmax only feeds it x <= 0.
// 2^(i/32) as double bits minus i<<47: the table of the exp2f-family reduction
// (exp(x) = 2^(k/32) * 2^(r/32)); entry i is the correctly rounded double of
// 2^(i/32) with the exponent contribution of i/32 taken out.
#define JY_EXP2_TABLE { \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull, \
}

// expf_libm with the table at `tab` (a kernel that calls it in bulk passes a copy in
// LDS: the constant-memory table is a global-memory load per call)
__host__ __device__ __forceinline__ float expf_tab(float x, const uint64_t* tab) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                      // |x| >= 88 or non-finite
        if (ux == 0xff800000u) return 0.0f;      // -inf
        if (abstop >= 0x7f8u) return x + x;      // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki & 31u];
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

__host__ __device__ __forceinline__ float expf_libm(float x) {
    static constexpr uint64_t kExp2Tab[32] = JY_EXP2_TABLE;
    return expf_tab(x, kExp2Tab);
}

// SiLU of libs/model_libs/silu/x86/x86_classic.txt:2-28 as GCC -O3 builds it with
// FMA: Cody-Waite reduction and the denominator contracted, explicit polynomial
// FMAs, 2^n by exponent bits, one correctly rounded division.
__host__ __device__ __forceinline__ float silu_ref(float vx) {
    float xa = 0.0f - vx;
    xa = xa > -87.0f ? xa : -87.0f;
    xa = xa < 88.0f ? xa : 88.0f;
    const float nf = __builtin_rintf(xa * 1.44269504088896341f);
    const float r = __builtin_fmaf(-nf, -2.12194440e-4f, __builtin_fmaf(-nf, 0.693359375f, xa));
    float p = __builtin_fmaf(1.0f / 720.0f, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float two_n = __builtin_bit_cast(float, (uint32_t)((int)nf + 127) << 23);
    return vx / __builtin_fmaf(p, two_n, 1.0f);
}

// SiLU of the elements past the last full group of 8 of the flattened gate buffer
// (libs/model_libs/silu/x86/x86_classic.txt:30-31): x / (1 + expf(-x)) with libm expf.
__host__ __device__ __forceinline__ float silu_tail(float vx) { return vx / (1.0f + expf_libm(-vx)); }

// silu of element e of a flattened gate buffer of n elements: the 8-wide form for the
// first n/8*8, the libm form for the rest, as the reference's silu(gate, gate, n)
__host__ __device__ __forceinline__ float silu_at(float vx, size_t e, size_t n) {
    return e < n / 8 * 8 ? silu_ref(vx) : silu_tail(vx);
}

// int8 absmax quantisation step of kv_pack_q8 / the Q quantisation in attention
// (libs/model_libs/attention/attention_q8.h:29-35): clamp to +-127, lrintf.
__host__ __device__ __forceinline__ int8_t quant_i8(float v, float inv) {
    float x = v * inv;
    x = x > 127.0f ? 127.0f : (x < -127.0f ? -127.0f : x);
    return (int8_t)(int)__builtin_rintf(x);
}

__host__ __device__ __forceinline__ float quant_inv(float amax) { return amax > 1e-8f ? 127.0f / amax : 0.0f; }
__host__ __device__ __forceinline__ float quant_scale(float amax) { return amax > 1e-8f ? amax / 127.0f : 0.0f; }

// Cross-lane moves within rows of 16 lanes by DPP (VALU, no LDS round trip): lane l
// receives the value of lane
//   0xB1  quad_perm [1,0,3,2]  l ^ 1
//   0x4E  quad_perm [2,3,0,1]  l ^ 2
//   0x120 + n  row_ror:n       (l - n) mod 16 of its row (so row_ror:12 gives l + 4)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
#else
    return v;  // host pass: never called
#endif
}

__device__ __forceinline__ float read_lane(float v, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
#else
    return v;  // host pass: never called
#endif
}

// Workgroup barrier that orders LDS only: global loads in flight stay in flight
// (__syncthreads also waits for every outstanding load of the calling wave).
__device__ __forceinline__ void lds_barrier() {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#endif
}

// Activation loads and stores: COH (one kernel whose workgroups hand each other data,
// possibly on other XCDs, whose L2 caches are not coherent with each other) reads and
// writes through to the agent-coherent level (sc1 on gfx950); otherwise plain accesses
// (the data was written by an earlier kernel: the kernel boundary makes it visible).
template <bool COH>
__device__ __forceinline__ float act_ld(const float* p) {
    if (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *p;
}
template <bool COH>
__device__ __forceinline__ void act_st(float* p, float v) {
    if (COH)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

// keys per slice of the split attention for nk live keys over ns slices (a multiple of 16)
static constexpr int SPL_MIN_CHUNK = 16;
__host__ __device__ __forceinline__ int split_chunk(int nk, int ns) {
    int c = (nk + ns - 1) / ns;
    c = (c + SPL_MIN_CHUNK - 1) / SPL_MIN_CHUNK * SPL_MIN_CHUNK;
    return c < SPL_MIN_CHUNK ? SPL_MIN_CHUNK : c;
}

// e^x from the hardware exp2 (v_exp_f32): about 1 ulp plus the rounding of x*log2(e),
// a relative error under 1e-6 for the |x| <= 20 that carry weight here
__device__ __forceinline__ float exp_hw(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
#else
    return x;  // host pass: never called
#endif
}

// maximum over the 64 lanes of a wave, in every lane (fmaxf: order-independent for
// the non-negative / finite values it is used on)
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));  // every lane: its row's maximum
    return fmaxf(fmaxf(read_lane(v, 0), read_lane(v, 16)), fmaxf(read_lane(v, 32), read_lane(v, 48)));
}

}  // namespace jy
