/*
 * jy_oracle.c — CPU oracle for jieyu's decode path.  TEST INFRASTRUCTURE ONLY
 * (what the GPU path is checked against; never part of the product).  See
 * jy_oracle.h for how it is pinned.
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf(), every other operation is rounded on its own, in the order the
 * reference's x86 AVX2+FMA path performs it.  Where the reference relies on
 * GCC contracting plain C into FMA (SiLU, scalar tails), the comment says so.
 */
#include "jy_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

float jyo_f16_to_f32(uint16_t h) {
    /* bit-exact half->float incl. subnormals (libs/date_libs/wmat.h:8-24) */
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {
            int k = 0;
            while (!(m & 0x400u)) { m <<= 1; k++; }
            bits = s | ((uint32_t)(113 - k) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | (m << 13);
    } else {
        bits = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float blk_scale(const uint8_t* b) { return jyo_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

/* libs/matmul_libs/matmul_q.h:22-33 (get_scale_min_k4): the 6-bit scale and min of
 * sub-block j of a Q4_K / Q5_K super-block */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

int jyo_block_elems(int type) { return type == JY_Q8_0 ? 32 : 256; }

int jyo_block_bytes(int type) {
    switch (type) {
        case JY_Q8_0: return 34;
        case JY_Q4_K: return 144;
        case JY_Q5_K: return 176;
        case JY_Q6_K: return 210;
        default: return 0;
    }
}

/* dequant_block (libs/matmul_libs/matmul_q.h:47-100; Q4_K through
 * libs/file_libs/q4/q4.h:8-35, whose AVX2+FMA form q4_fma.txt computes
 * fma(q, d*sc, -(dmin*m))).  Every product here is exact in float: d*sc and
 * dmin*m are an fp16 times a 6-bit integer (<= 17 significant bits), d1*q adds
 * 4-5 bits, and Q6_K's (d*sc)*q is 11 + 8 + 6 bits.  So the fused and unfused
 * forms GCC might emit agree: Q4_K / Q5_K values are the one rounding of
 * d1*q - n1, Q6_K values are exact. */
void jyo_dequant_block(int type, const uint8_t* b, float* dst) {
    switch (type) {
        case JY_Q8_0: {
            const float d = blk_scale(b);
            for (int l = 0; l < 32; l++) dst[l] = (float)(int8_t)b[2 + l] * d;
            return;
        }
        case JY_Q4_K:
        case JY_Q5_K: {
            const float d = blk_scale(b), dmin = blk_scale(b + 2);
            const uint8_t* sc = b + 4;
            const uint8_t* qh = b + 16; /* Q5_K only */
            const uint8_t* qs = type == JY_Q4_K ? b + 16 : b + 48;
            for (int g = 0; g < 4; g++) {
                for (int half = 0; half < 2; half++) {
                    const int j = 2 * g + half;
                    int s, m;
                    scale_min_k4(j, sc, &s, &m);
                    const float d1 = d * (float)s, n1 = dmin * (float)m;
                    for (int l = 0; l < 32; l++) {
                        int q = half ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 0xF);
                        if (type == JY_Q5_K && (qh[l] >> j) & 1) q += 16;
                        dst[64 * g + 32 * half + l] = fmaf((float)q, d1, -n1);
                    }
                }
            }
            return;
        }
        case JY_Q6_K: {
            const uint8_t* ql = b;
            const uint8_t* qh = b + 128;
            const int8_t* sc = (const int8_t*)(b + 192);
            const float d = blk_scale(b + 208);
            for (int nn = 0; nn < 2; nn++) {
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    dst[128 * nn + l] = (d * (float)sc[is]) * (float)q1;
                    dst[128 * nn + l + 32] = (d * (float)sc[is + 2]) * (float)q2;
                    dst[128 * nn + l + 64] = (d * (float)sc[is + 4]) * (float)q3;
                    dst[128 * nn + l + 96] = (d * (float)sc[is + 6]) * (float)q4;
                }
                ql += 64;
                qh += 32;
                sc += 8;
            }
            return;
        }
        default: return;
    }
}

/* libs/matmul_libs/matmul_q.h:111-132: four 8-wide FMA accumulators = 32 virtual
 * lanes, lane L takes element 32c+L of every 32-element step c in order, each
 * block dequantized first (dequant_block above). */
float jyo_q_row_dot(const float* x, const uint8_t* row, int type, int k) {
    float a[32], blk[256];
    for (int L = 0; L < 32; L++) a[L] = 0.0f;
    const int be = jyo_block_elems(type), bb = jyo_block_bytes(type), nb = k / be;
    for (int b = 0; b < nb; b++) {
        jyo_dequant_block(type, row + (size_t)b * bb, blk);
        for (int l = 0; l < be; l++) a[l & 31] = fmaf(x[(size_t)b * be + l], blk[l], a[l & 31]);
    }
    /* matmul_q.h:127-131: (s0+s1)+(s2+s3), then 128-bit halves, then two hadds */
    float s[8], r[4];
    for (int i = 0; i < 8; i++) s[i] = (a[i] + a[8 + i]) + (a[16 + i] + a[24 + i]);
    for (int i = 0; i < 4; i++) r[i] = s[i] + s[4 + i];
    return (r[0] + r[1]) + (r[2] + r[3]);
}

float jyo_q8_row_dot(const float* x, const uint8_t* row, int k) { return jyo_q_row_dot(x, row, JY_Q8_0, k); }

void jyo_matmul_q(const float* a, const uint8_t* w, float* c, int m, int n, int k, int type) {
    const int be = jyo_block_elems(type), bb = jyo_block_bytes(type), nb = k / be;
    const size_t rbytes = (size_t)nb * bb;
    if (m == 1) { /* matmul_q.h:139-143 (AVX2+FMA host) */
#pragma omp parallel for schedule(static)
        for (int j = 0; j < n; j++) c[j] = jyo_q_row_dot(a, w + (size_t)j * rbytes, type, k);
        return;
    }
    /* matmul_q.h:145-161: sequential k, product and sum rounded separately (no FMA:
     * the generic lambda is compiled for baseline x86-64) */
#pragma omp parallel
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)m);
        float blk[256];
#pragma omp for schedule(static)
        for (int j = 0; j < n; j++) {
            const uint8_t* row = w + (size_t)j * rbytes;
            for (int i = 0; i < m; i++) acc[i] = 0.0f;
            for (int b = 0; b < nb; b++) {
                jyo_dequant_block(type, row + (size_t)b * bb, blk);
                for (int l = 0; l < be; l++) {
                    const float bv = blk[l];
                    const size_t off = (size_t)b * be + (size_t)l;
                    for (int i = 0; i < m; i++) {
                        const float p = a[(size_t)i * k + off] * bv;
                        acc[i] = acc[i] + p;
                    }
                }
            }
            for (int i = 0; i < m; i++) c[(size_t)i * n + j] = acc[i];
        }
        free(acc);
    }
}

void jyo_matmul_q8(const float* a, const uint8_t* w, float* c, int m, int n, int k) {
    jyo_matmul_q(a, w, c, m, n, k, JY_Q8_0);
}

/* libs/matmul_libs/matmul.h:7-8 + x86/x86_classic.txt:2-16: C = 0, then for p in
 * order C[i][j] = fma(A[i][p], B[p][j], C[i][j]); the n%8 tail is the same
 * expression contracted by GCC. */
void jyo_matmul_f32(int m, int n, int k, const float* A, const float* B, float* C) {
    memset(C, 0, sizeof(float) * (size_t)m * (size_t)n);
#pragma omp parallel for schedule(static) if (m >= 4)
    for (int i = 0; i < m; i++) {
        float* crow = C + (size_t)i * n;
        const float* arow = A + (size_t)i * k;
        for (int p = 0; p < k; p++) {
            const float av = arow[p];
            const float* brow = B + (size_t)p * n;
            for (int j = 0; j < n; j++) crow[j] = fmaf(av, brow[j], crow[j]);
        }
    }
}

/* libs/model_libs/wmat_kernel.h:12-15 + libs/matmul_libs/matmul_f16.h:19-41: C = 0
 * (memset), then for p in order C[i][j] = fma(A[i][p], (float)B[p][j], C[i][j]);
 * half -> float is exact and the n%8 tail is the same expression contracted by
 * GCC (the function is compiled with fma). */
void jyo_matmul_f16(int m, int n, int k, const float* A, const uint16_t* B, float* C) {
    memset(C, 0, sizeof(float) * (size_t)m * (size_t)n);
#pragma omp parallel for schedule(static) if (m >= 4)
    for (int i = 0; i < m; i++) {
        float* crow = C + (size_t)i * n;
        const float* arow = A + (size_t)i * k;
        for (int p = 0; p < k; p++) {
            const float av = arow[p];
            const uint16_t* brow = B + (size_t)p * n;
            for (int j = 0; j < n; j++) crow[j] = fmaf(av, jyo_f16_to_f32(brow[j]), crow[j]);
        }
    }
}

void jyo_matmul_w(const jy_wmat* w, int m, int n, int k, const float* A, float* C) {
    if (w->type == JY_F32)
        jyo_matmul_f32(m, n, k, A, (const float*)w->data, C);
    else if (w->type == JY_F16)
        jyo_matmul_f16(m, n, k, A, (const uint16_t*)w->data, C);
    else
        jyo_matmul_q(A, (const uint8_t*)w->data, C, m, n, k, w->type);
}

/* wmat_row (libs/model_libs/wmat_kernel.h:18-29): f32 copy, f16 converted, or the
 * row's blocks dequantized */
void jyo_embed_row(const jy_wmat* w, int id, int width, float* dst) {
    if (w->type == JY_F32) {
        memcpy(dst, (const float*)w->data + (size_t)id * width, sizeof(float) * (size_t)width);
    } else if (w->type == JY_F16) {
        const uint16_t* row = (const uint16_t*)w->data + (size_t)id * width;
        for (int i = 0; i < width; i++) dst[i] = jyo_f16_to_f32(row[i]);
    } else {
        const int be = jyo_block_elems(w->type), bb = jyo_block_bytes(w->type), nb = width / be;
        const uint8_t* row = (const uint8_t*)w->data + (size_t)id * nb * bb;
        for (int b = 0; b < nb; b++) jyo_dequant_block(w->type, row + (size_t)b * bb, dst + (size_t)b * be);
    }
}

/* rmsnorm/x86/x86_classic.txt:2-26: 16 FMA lanes over x^2 (an 8-wide remainder pass
 * feeds lanes 0..7), reduction ((v0+v1) -> halves -> two hadds), then the scalar
 * tail of t < 8 elements (:15), then y = (x*scale)*w.  GCC 11 -O3 builds that
 * tail loop as an in-order vector reduction: when t >= 4 the first four squares
 * are rounded products added in order, the rest are contracted to FMAs. */
void jyo_rmsnorm(const float* x, float* y, const float* w, int n, float eps) {
    float v[16];
    for (int l = 0; l < 16; l++) v[l] = 0.0f;
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) v[l] = fmaf(x[i + l], x[i + l], v[l]);
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) v[l] = fmaf(x[i + l], x[i + l], v[l]);
    float s[8], t[4];
    for (int l = 0; l < 8; l++) s[l] = v[l] + v[8 + l];
    for (int l = 0; l < 4; l++) t[l] = s[l] + s[4 + l];
    float ss = (t[0] + t[1]) + (t[2] + t[3]);
    if (n - i >= 4)
        for (const int e = i + 4; i < e; i++) ss = ss + x[i] * x[i];
    for (; i < n; i++) ss = fmaf(x[i], x[i], ss);
    const float den = ss / (float)n + eps;
    if (den <= 0.0f) {
        for (int k = 0; k < n; k++) y[k] = 0.0f;
        return;
    }
    const float scale = 1.0f / sqrtf(den);
    for (int k = 0; k < n; k++) y[k] = (x[k] * scale) * w[k];
}

/* libs/date_libs/date.h:58-65 (float arithmetic, host libm) */
void jyo_rope_table(int max_seq, int head_dim, float theta, float* cos_t, float* sin_t) {
    const int half = head_dim / 2;
    for (int i = 0; i < max_seq; i++)
        for (int j = 0; j < half; j++) {
            const float freq = 1.0f / powf(theta, 2.0f * (float)j / (float)head_dim);
            const float ang = (float)i * freq;
            cos_t[(size_t)i * half + j] = cosf(ang);
            sin_t[(size_t)i * half + j] = sinf(ang);
        }
}

/* rope/x86/x86_classic.txt:10-29.  Each group of 8 pairs is rotated with
 *   y0 = fma(x0, c, -(x1*s)), y1 = fma(x0, s, x1*c)
 * and stored back through unpacklo/unpackhi, which lands rotated pairs (4,5) of
 * the group in slots (2,3) and pairs (2,3) in slots (4,5).  Q and K get the same
 * permutation, so q.k is unchanged; the stored K values follow it.  Remainder
 * pairs (:30-35) use the same expressions, contracted by GCC. */
void jyo_rope(float* q, int seq, int start_pos, int num_heads, int head_dim, const float* cos_t,
              const float* sin_t) {
    static const int slot[8] = {0, 1, 4, 5, 2, 3, 6, 7}; /* source pair -> destination pair */
    const int half = head_dim / 2;
    for (int r = 0; r < seq; r++) {
        const float* c = cos_t + (size_t)(start_pos + r) * half;
        const float* s = sin_t + (size_t)(start_pos + r) * half;
        for (int h = 0; h < num_heads; h++) {
            float* qh = q + ((size_t)r * num_heads + h) * head_dim;
            int i = 0;
            for (; i + 8 <= half; i += 8) {
                float y[16];
                for (int m = 0; m < 8; m++) {
                    const float x0 = qh[2 * (i + m)], x1 = qh[2 * (i + m) + 1];
                    const float cc = c[i + m], sn = s[i + m];
                    y[2 * slot[m]] = fmaf(x0, cc, -(x1 * sn));
                    y[2 * slot[m] + 1] = fmaf(x0, sn, x1 * cc);
                }
                memcpy(qh + 2 * i, y, sizeof(y));
            }
            for (; i < half; i++) {
                const float x0 = qh[2 * i], x1 = qh[2 * i + 1];
                qh[2 * i] = fmaf(x0, c[i], -(x1 * s[i]));
                qh[2 * i + 1] = fmaf(x0, s[i], x1 * c[i]);
            }
        }
    }
}

/* attention_q8.h:20-37: per (row, head) absmax int8, lrintf (ties-to-even) */
void jyo_kv_pack(const float* src, int8_t* dst, float* sc, int heads, int hd, int n) {
    for (int i = 0; i < n; i++)
        for (int h = 0; h < heads; h++) {
            const float* s = src + ((size_t)i * heads + h) * hd;
            int8_t* d = dst + ((size_t)i * heads + h) * hd;
            float amax = 0.0f;
            for (int k = 0; k < hd; k++) {
                const float a = fabsf(s[k]);
                if (a > amax) amax = a;
            }
            const float inv = amax > 1e-8f ? 127.0f / amax : 0.0f;
            sc[(size_t)i * heads + h] = amax > 1e-8f ? amax / 127.0f : 0.0f;
            for (int k = 0; k < hd; k++) {
                float x = s[k] * inv;
                x = x > 127.0f ? 127.0f : (x < -127.0f ? -127.0f : x);
                d[k] = (int8_t)lrintf(x);
            }
        }
}

int jyo_kv_init(jyo_kv* kv, int num_layers, int max_seq, int num_kv_heads, int head_dim) {
    memset(kv, 0, sizeof(*kv));
    const size_t n = (size_t)num_layers * max_seq * num_kv_heads * head_dim;
    const size_t rows = (size_t)num_layers * max_seq * num_kv_heads;
    kv->k = (int8_t*)calloc(n ? n : 1, 1);
    kv->v = (int8_t*)calloc(n ? n : 1, 1);
    kv->ks = (float*)calloc(rows ? rows : 1, sizeof(float));
    kv->vs = (float*)calloc(rows ? rows : 1, sizeof(float));
    if (!kv->k || !kv->v || !kv->ks || !kv->vs) {
        jyo_kv_free(kv);
        return -1;
    }
    kv->num_layers = num_layers;
    kv->max_seq = max_seq;
    kv->num_kv_heads = num_kv_heads;
    kv->head_dim = head_dim;
    return 0;
}

void jyo_kv_free(jyo_kv* kv) {
    free(kv->k);
    free(kv->v);
    free(kv->ks);
    free(kv->vs);
    memset(kv, 0, sizeof(*kv));
}

/* attention/x86/x86_classic.txt:1-73 (AVX2+FMA): pack K,V, then per q-head
 * (kv head = h / group): Q -> int8, exact int32 q.k, score = dot*((ks*qsc)*scale),
 * strict max from -1e30, expf, ascending float sum, normalise, and the PV chain
 * o[d] = fma(p_j*vs_j, (float)v8, o[d]) in ascending j. */
int jyo_attention(float* Q, const float* K, const float* V, float* out, int seq, int start_pos,
                  int num_heads, int num_kv_heads, int head_dim, int8_t* kc, float* ksc, int8_t* vc,
                  float* vsc, int cap) {
    if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || seq <= 0 || start_pos < 0) return -1;
    if ((size_t)start_pos + (size_t)seq > (size_t)cap) return -1;
    const int kv_dim = num_kv_heads * head_dim;
    jyo_kv_pack(K, kc + (size_t)start_pos * kv_dim, ksc + (size_t)start_pos * num_kv_heads, num_kv_heads,
                head_dim, seq);
    jyo_kv_pack(V, vc + (size_t)start_pos * kv_dim, vsc + (size_t)start_pos * num_kv_heads, num_kv_heads,
                head_dim, seq);
    const int group = num_heads / num_kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < num_heads; h++) {
        float* scores = (float*)malloc(sizeof(float) * ((size_t)start_pos + seq));
        int8_t* q8 = (int8_t*)malloc((size_t)head_dim);
        const int kvh = h / group;
        for (int i = 0; i < seq; i++) {
            const int p = start_pos + i;
            const float* q = Q + ((size_t)i * num_heads + h) * head_dim;
            float amax = 0.0f;
            for (int d = 0; d < head_dim; d++) {
                const float a = fabsf(q[d]);
                if (a > amax) amax = a;
            }
            const float qinv = amax > 1e-8f ? 127.0f / amax : 0.0f;
            const float qsc = amax > 1e-8f ? amax / 127.0f : 0.0f;
            for (int d = 0; d < head_dim; d++) {
                float x = q[d] * qinv;
                x = x > 127.0f ? 127.0f : (x < -127.0f ? -127.0f : x);
                q8[d] = (int8_t)lrintf(x);
            }
            float mx = -1e30f;
            for (int j = 0; j <= p; j++) {
                const int8_t* kr = kc + ((size_t)j * num_kv_heads + kvh) * head_dim;
                const float f = (ksc[(size_t)j * num_kv_heads + kvh] * qsc) * scale;
                int32_t dot = 0;
                for (int d = 0; d < head_dim; d++) dot += (int32_t)q8[d] * (int32_t)kr[d];
                const float dt = (float)dot * f;
                scores[j] = dt;
                if (dt > mx) mx = dt;
            }
            float sum = 0.0f;
            for (int j = 0; j <= p; j++) {
                scores[j] = expf(scores[j] - mx);
                sum += scores[j];
            }
            const float inv_sum = 1.0f / sum;
            for (int j = 0; j <= p; j++) scores[j] *= inv_sum;
            float* o = out + ((size_t)i * num_heads + h) * head_dim;
            for (int d = 0; d < head_dim; d++) o[d] = 0.0f;
            for (int j = 0; j <= p; j++) {
                const int8_t* vr = vc + ((size_t)j * num_kv_heads + kvh) * head_dim;
                const float pr = scores[j] * vsc[(size_t)j * num_kv_heads + kvh];
                for (int d = 0; d < head_dim; d++) o[d] = fmaf(pr, (float)vr[d], o[d]);
            }
        }
        free(scores);
        free(q8);
    }
    return 0;
}

/* silu/x86/x86_classic.txt:2-28 as GCC -O3 compiles it with FMA enabled: the
 * Cody-Waite reduction and the denominator are contracted, the polynomial FMAs
 * are explicit.  Remainder elements (:30-31) use libm expf. */
void jyo_silu(const float* x, float* y, int n) {
    const int nv = n / 8 * 8;
#pragma omp parallel for schedule(static) if (n >= 8192)
    for (int i = 0; i < nv; i++) {
        const float vx = x[i];
        float xa = 0.0f - vx;
        xa = xa > -87.0f ? xa : -87.0f; /* _mm256_max_ps(xa, -87): second operand on NaN */
        xa = xa < 88.0f ? xa : 88.0f;
        const float nf = rintf(xa * 1.44269504088896341f);
        const float r = fmaf(-nf, -2.12194440e-4f, fmaf(-nf, 0.693359375f, xa));
        float p = fmaf(1.0f / 720.0f, r, 1.0f / 120.0f);
        p = fmaf(p, r, 1.0f / 24.0f);
        p = fmaf(p, r, 1.0f / 6.0f);
        p = fmaf(p, r, 0.5f);
        p = fmaf(p, r, 1.0f);
        p = fmaf(p, r, 1.0f);
        const uint32_t eb = (uint32_t)((int32_t)nf + 127) << 23;
        float two_n;
        memcpy(&two_n, &eb, 4);
        y[i] = vx / fmaf(p, two_n, 1.0f);
    }
    for (int i = nv; i < n; i++) y[i] = x[i] / (1.0f + expf(-x[i]));
}

/* libs/model_libs/transformer_layer.h:10-90 */
int jyo_transformer_layer(float* X, const jy_layer_weights* w, const float* cos_t, const float* sin_t,
                          int seq, int hidden, int num_heads, int num_kv_heads, int head_dim,
                          int intermediate, int start_pos, jyo_kv* kv, int layer, float eps) {
    const int qd = num_heads * head_dim, kvd = num_kv_heads * head_dim;
    const size_t S = (size_t)seq;
    float* xn = (float*)malloc(sizeof(float) * S * hidden);
    float* Qb = (float*)malloc(sizeof(float) * S * qd);
    float* Kb = (float*)malloc(sizeof(float) * S * kvd);
    float* Vb = (float*)malloc(sizeof(float) * S * kvd);
    float* att = (float*)malloc(sizeof(float) * S * qd);
    float* proj = (float*)malloc(sizeof(float) * S * hidden);
    float* gate = (float*)malloc(sizeof(float) * S * intermediate);
    float* up = (float*)malloc(sizeof(float) * S * intermediate);
    int rc = -1;
    if (!xn || !Qb || !Kb || !Vb || !att || !proj || !gate || !up) goto done;

    for (int i = 0; i < seq; i++)
        jyo_rmsnorm(X + (size_t)i * hidden, xn + (size_t)i * hidden, w->rms1_weight, hidden, eps);
    jyo_matmul_w(&w->Wq, seq, qd, hidden, xn, Qb);
    jyo_matmul_w(&w->Wk, seq, kvd, hidden, xn, Kb);
    jyo_matmul_w(&w->Wv, seq, kvd, hidden, xn, Vb);
    if (w->bq)
        for (size_t i = 0; i < S; i++)
            for (int j = 0; j < qd; j++) Qb[i * qd + j] += w->bq[j];
    if (w->bk)
        for (size_t i = 0; i < S; i++)
            for (int j = 0; j < kvd; j++) Kb[i * kvd + j] += w->bk[j];
    if (w->bv)
        for (size_t i = 0; i < S; i++)
            for (int j = 0; j < kvd; j++) Vb[i * kvd + j] += w->bv[j];
    jyo_rope(Qb, seq, start_pos, num_heads, head_dim, cos_t, sin_t);
    jyo_rope(Kb, seq, start_pos, num_kv_heads, head_dim, cos_t, sin_t);
    {
        const size_t lo = (size_t)layer * kv->max_seq;
        if (jyo_attention(Qb, Kb, Vb, att, seq, start_pos, num_heads, num_kv_heads, head_dim,
                          kv->k + lo * kvd, kv->ks + lo * num_kv_heads, kv->v + lo * kvd,
                          kv->vs + lo * num_kv_heads, kv->max_seq))
            goto done;
    }
    jyo_matmul_w(&w->Wo, seq, hidden, qd, att, proj);
    for (size_t i = 0; i < S * hidden; i++) X[i] += proj[i];
    for (int i = 0; i < seq; i++)
        jyo_rmsnorm(X + (size_t)i * hidden, xn + (size_t)i * hidden, w->rms2_weight, hidden, eps);
    /* libs/model_libs/ffn/ffn.h:7-19 */
    jyo_matmul_w(&w->W1, seq, intermediate, hidden, xn, gate);
    jyo_matmul_w(&w->W3, seq, intermediate, hidden, xn, up);
    jyo_silu(gate, gate, seq * intermediate);
    for (size_t i = 0; i < S * intermediate; i++) gate[i] = gate[i] * up[i];
    jyo_matmul_w(&w->W2, seq, hidden, intermediate, gate, proj);
    for (size_t i = 0; i < S * hidden; i++) X[i] += proj[i];
    rc = 0;
done:
    free(xn); free(Qb); free(Kb); free(Vb); free(att); free(proj); free(gate); free(up);
    return rc;
}

/* libs/model_libs/forward.h:47-96 */
int jyo_forward_cached(const jy_model_desc* m, float* X, const float* cos_t, const float* sin_t, int seq,
                       int start_pos, jyo_kv* kv, float* layer_out) {
    if (kv->num_layers < m->num_layers || kv->num_kv_heads != m->num_kv_heads || kv->head_dim != m->head_dim)
        return -1;
    if (start_pos < 0 || (size_t)start_pos + (size_t)seq > (size_t)kv->max_seq) return -1;
    const int H = m->hidden;
    for (int l = 0; l < m->num_layers; l++) {
        if (jyo_transformer_layer(X, &m->layers[l], cos_t, sin_t, seq, H, m->num_heads, m->num_kv_heads,
                                  m->head_dim, m->intermediate, start_pos, kv, l, 1e-5f))
            return -1;
        if (layer_out) memcpy(layer_out + (size_t)l * seq * H, X, sizeof(float) * (size_t)seq * H);
    }
    float* xn = (float*)malloc(sizeof(float) * (size_t)seq * H);
    if (!xn) return -1;
    for (int i = 0; i < seq; i++)
        jyo_rmsnorm(X + (size_t)i * H, xn + (size_t)i * H, m->final_rms_weight, H, 1e-5f);
    memcpy(X, xn, sizeof(float) * (size_t)seq * H);
    free(xn);
    kv->current_len = start_pos + seq;
    return 0;
}

/* libs/model_libs/generate.h:9-112 */
int jyo_generate(const jy_model_desc* m, const int* prompt_ids, int prompt_len, const int* eos_ids,
                 int num_eos, const float* cos_t, const float* sin_t, int max_seq, int max_new,
                 float temperature, float repetition_penalty, int* out_ids, jyo_kv* kv_in,
                 float* last_logits) {
    if (prompt_len <= 0 || prompt_len > max_seq) return 0;
    jyo_kv own;
    jyo_kv* kv = kv_in;
    if (!kv) {
        if (jyo_kv_init(&own, m->num_layers, max_seq, m->num_kv_heads, m->head_dim)) return -1;
        kv = &own;
    }
    if (kv->num_layers < m->num_layers || kv->max_seq < max_seq || kv->num_kv_heads != m->num_kv_heads ||
        kv->head_dim != m->head_dim) {
        if (!kv_in) jyo_kv_free(&own);
        return -1;
    }
    for (int i = 0; i < prompt_len; i++) out_ids[i] = prompt_ids[i];
    kv->current_len = 0;
    if (max_new <= 0) {
        if (!kv_in) jyo_kv_free(&own);
        return prompt_len;
    }
    const int H = m->hidden, V = m->vocab_size;
    float* X = (float*)malloc(sizeof(float) * (size_t)max_seq * H);
    float* logits = (float*)calloc((size_t)V, sizeof(float));
    unsigned rng = 12345u;
    int len = prompt_len, seq = prompt_len;
    for (int step = 0; step < max_new && len < max_seq; step++) {
        const int start_pos = len - seq;
        for (int i = 0; i < seq; i++) jyo_embed_row(&m->embed, out_ids[start_pos + i], H, X + (size_t)i * H);
        if (jyo_forward_cached(m, X, cos_t, sin_t, seq, start_pos, kv, NULL)) {
            len = -1;
            break;
        }
        jyo_matmul_w(&m->lm_head, 1, V, H, X + (size_t)(seq - 1) * H, logits);
        if (repetition_penalty != 1.0f)
            for (int i = prompt_len; i < len; i++) {
                const int id = out_ids[i];
                if (id >= 0 && id < V)
                    logits[id] = logits[id] > 0.0f ? logits[id] / repetition_penalty : logits[id] * repetition_penalty;
            }
        if (last_logits) memcpy(last_logits, logits, sizeof(float) * (size_t)V);
        int next = 0;
        if (temperature <= 0.0f) {
            for (int v = 1; v < V; v++)
                if (logits[v] > logits[next]) next = v;
        } else {
            float mx = logits[0];
            for (int v = 1; v < V; v++)
                if (logits[v] > mx) mx = logits[v];
            double sum = 0.0;
            for (int v = 0; v < V; v++) {
                logits[v] = expf((logits[v] - mx) / temperature);
                sum += logits[v];
            }
            rng = rng * 1664525u + 1013904223u;
            double r = (double)(rng >> 8) / 16777216.0 * sum;
            next = V - 1;
            for (int v = 0; v < V; v++) {
                r -= logits[v];
                if (r <= 0.0) {
                    next = v;
                    break;
                }
            }
        }
        out_ids[len++] = next;
        seq = 1;
        int stop = 0;
        if (eos_ids)
            for (int e = 0; e < num_eos; e++)
                if (next == eos_ids[e]) stop = 1;
        if (stop) break;
    }
    free(X);
    free(logits);
    if (!kv_in) jyo_kv_free(&own);
    return len;
}
