// Host build of the device arithmetic in jieyu_amd/csrc/jy_device.h.  TEST
// INFRASTRUCTURE ONLY: the helpers there are __host__ __device__, so the same
// source compiles for x86 here and is checked exhaustively against the host libm
// and the C oracle (tests/test_device_math.py).  The GPU build of the same source
// is covered by the GPU parity tests.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <thread>
#include <vector>

#include "../jieyu_amd/csrc/jy_device.h"

#define JYDM_API extern "C" __attribute__((visibility("default")))

static inline uint32_t fbits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// Number of 32-bit patterns lo, lo+step, ... below hi whose expf_libm result
// differs in bits from the host libm's expf (NaN results compare as equal when
// both are NaN).  The first mismatching pattern goes to *first (unchanged when
// there is none).
JYDM_API uint64_t jydm_expf_mismatches(uint64_t lo, uint64_t hi, uint64_t step, uint32_t* first) {
    const uint64_t count = hi > lo ? (hi - lo + step - 1) / step : 0;
    unsigned nt = std::thread::hardware_concurrency();
    nt = nt < 1 ? 1 : (nt > 16 ? 16 : nt);
    std::vector<uint64_t> bad(nt, 0), first_bad(nt, UINT64_MAX);
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; t++)
        pool.emplace_back([&, t] {
            for (uint64_t j = count * t / nt; j < count * (t + 1) / nt; j++) {
                const uint64_t i = lo + j * step;
                const uint32_t u = (uint32_t)i;
                float x;
                memcpy(&x, &u, 4);
                const float a = jy::expf_libm(x);
                const float b = expf(x);
                if (fbits(a) != fbits(b) && !(isnan(a) && isnan(b))) {
                    if (!bad[t]) first_bad[t] = i;
                    bad[t]++;
                }
            }
        });
    uint64_t total = 0, fb = UINT64_MAX;
    for (unsigned t = 0; t < nt; t++) {
        pool[t].join();
        total += bad[t];
        fb = first_bad[t] < fb ? first_bad[t] : fb;
    }
    if (total && first) *first = (uint32_t)fb;
    return total;
}

JYDM_API float jydm_expf(float x) { return jy::expf_libm(x); }

JYDM_API void jydm_silu(const float* x, float* y, int n) {
    for (int i = 0; i < n; i++) y[i] = jy::silu_ref(x[i]);
}

JYDM_API void jydm_half_to_float(const uint16_t* h, float* y, int n) {
    for (int i = 0; i < n; i++) y[i] = jy::half_to_float(h[i]);
}

JYDM_API void jydm_quant(const float* v, int n, int8_t* q, float* scale) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float inv = jy::quant_inv(amax);
    *scale = jy::quant_scale(amax);
    for (int i = 0; i < n; i++) q[i] = jy::quant_i8(v[i], inv);
}
