#define _POSIX_C_SOURCE 200809L
/*
 * jy_synth.c — deterministic synthetic models for the decode path.
 *
 * Counter-based generation: element i of stream s under seed S depends only on
 * (S, s, i), so the same bytes come out for any thread count and on any host
 * with the same libm.  The logical weight W[out][in] is generated in
 * out-major order for every storage type, then stored in the layout jieyu
 * binds for that type (include/jieyu_model.h).
 */
#include "jieyu_synth.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(mix64(seed) ^ (stream * 0xD6E8FEB86659FD93ull));
}

static inline uint64_t draw(uint64_t key, uint64_t i) {
    return mix64(key ^ (i * 0xA0761D6478BD642Full));
}

/* (0, 1) from the top 53 bits */
static inline double unit_open(uint64_t b) {
    return ((double)(b >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

/* Box-Muller pair k of a stream -> z[0], z[1] ~ N(0,1) */
static inline void normal_pair(uint64_t key, uint64_t k, double* z0, double* z1) {
    const double u1 = unit_open(draw(key, 2 * k));
    const double u2 = unit_open(draw(key, 2 * k + 1));
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586476925286766559 * u2;
    *z0 = r * cos(t);
    *z1 = r * sin(t);
}

void jysyn_normal_fill(uint64_t seed, uint64_t stream, float std, float* out, size_t n) {
    const uint64_t key = stream_key(seed, stream);
    const long long npair = (long long)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (long long k = 0; k < npair; k++) {
        double z0, z1;
        normal_pair(key, (uint64_t)k, &z0, &z1);
        const size_t i = (size_t)k * 2;
        out[i] = (float)(std * z0);
        if (i + 1 < n) out[i + 1] = (float)(std * z1);
    }
}

void jysyn_uniform_int_fill(uint64_t seed, uint64_t stream, int lo, int hi, int* out, size_t n) {
    const uint64_t key = stream_key(seed, stream);
    const uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (size_t i = 0; i < n; i++) out[i] = (int)((int64_t)lo + (int64_t)(draw(key, i) % span));
}

void jysyn_uniform_fill(uint64_t seed, uint64_t stream, float lo, float hi, float* out, size_t n) {
    const uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++)
        out[i] = (float)((double)lo + ((double)hi - (double)lo) * unit_open(draw(key, (uint64_t)i)));
}

static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t jysyn_f32_to_f16(float f) {
    const uint32_t x = fbits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) { /* result is subnormal (or zero) in half */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 126 - (int)e; /* value = m * 2^(e-150); half ulp 2^-24 -> q = m >> (126-e) */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((ax - 0x38000000u) >> 13);  /* rebias exponent 127 -> 15 */
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float jysyn_f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return bitsf(s);
        int k = 0;
        while (!(m & 0x400u)) { m <<= 1; k++; }
        return bitsf(s | ((uint32_t)(113 - k) << 23) | ((m & 0x3FFu) << 13));
    }
    if (e == 31) return bitsf(s | 0x7F800000u | (m << 13));
    return bitsf(s | ((e + 112u) << 23) | (m << 13));
}

static void quant_block(const float* x, uint8_t* out) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float a = fabsf(x[j]);
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = jysyn_f32_to_f16(d);
    out[0] = (uint8_t)(dh & 0xFF);
    out[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; j++) out[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

void jysyn_quantize_q8_0(const float* x, uint8_t* out, size_t n) {
    const long long nb = (long long)(n / 32);
#pragma omp parallel for schedule(static)
    for (long long b = 0; b < nb; b++) quant_block(x + b * 32, out + b * 34);
}

/* ---- model construction ---------------------------------------------- */

enum { S_EMBED = 1, S_LMHEAD = 2, S_FINAL = 3, S_LAYER0 = 16 };
enum { L_RMS1 = 0, L_WQ, L_WK, L_WV, L_WO, L_BQ, L_BK, L_BV, L_RMS2, L_W1, L_W2, L_W3, L_NSLOT = 16 };

static uint64_t layer_stream(int l, int slot) { return (uint64_t)S_LAYER0 + (uint64_t)l * L_NSLOT + (uint64_t)slot; }

static size_t align64(size_t x) { return (x + 63) & ~(size_t)63; }

static size_t wbytes(int type, size_t rows, size_t cols) {
    return type == JY_Q8_0 ? rows * (cols / 32) * 34 : rows * cols * 4;
}

/* W[out=rows][in=cols] ~ N(0,std): Q8_0 rows as stored, or f32 transposed to [in][out]. */
static void fill_matrix(uint64_t seed, uint64_t stream, float std, int type, size_t rows, size_t cols,
                        int f32_row_major, void* dst) {
    const uint64_t key = stream_key(seed, stream);
    if (type == JY_Q8_0) {
        const size_t nb = cols / 32;
        uint8_t* q = (uint8_t*)dst;
#pragma omp parallel for schedule(static)
        for (long long r = 0; r < (long long)rows; r++) {
            float blk[32];
            for (size_t b = 0; b < nb; b++) {
                const uint64_t base = ((uint64_t)r * cols + b * 32) / 2;
                for (int j = 0; j < 16; j++) {
                    double z0, z1;
                    normal_pair(key, base + (uint64_t)j, &z0, &z1);
                    blk[2 * j] = (float)(std * z0);
                    blk[2 * j + 1] = (float)(std * z1);
                }
                quant_block(blk, q + ((size_t)r * nb + b) * 34);
            }
        }
    } else {
        float* f = (float*)dst;
#pragma omp parallel for schedule(static)
        for (long long r = 0; r < (long long)rows; r++) {
            for (size_t c = 0; c < cols; c += 2) {
                double z0, z1;
                normal_pair(key, ((uint64_t)r * cols + c) / 2, &z0, &z1);
                const float v0 = (float)(std * z0), v1 = (float)(std * z1);
                if (f32_row_major) {
                    f[(size_t)r * cols + c] = v0;
                    f[(size_t)r * cols + c + 1] = v1;
                } else {
                    f[c * rows + (size_t)r] = v0;
                    f[(c + 1) * rows + (size_t)r] = v1;
                }
            }
        }
    }
}

static void fill_norm(uint64_t seed, uint64_t stream, float std, float* dst, size_t n) {
    jysyn_normal_fill(seed, stream, std, dst, n);
    for (size_t i = 0; i < n; i++) dst[i] = 1.0f + dst[i];
}

int jysyn_create(const jy_synth_config* c, jy_synth_model** out) {
    if (out) *out = NULL;
    if (!c || !out) return -1;
    if (c->num_layers <= 0 || c->hidden <= 0 || c->num_heads <= 0 || c->num_kv_heads <= 0 ||
        c->head_dim <= 0 || c->intermediate <= 0 || c->vocab_size <= 0)
        return -1;
    if (c->wtype != JY_F32 && c->wtype != JY_Q8_0) return -1;
    if (c->num_heads % c->num_kv_heads) return -1;
    const size_t d = (size_t)c->hidden, q = (size_t)c->num_heads * c->head_dim,
                 kv = (size_t)c->num_kv_heads * c->head_dim, F = (size_t)c->intermediate,
                 V = (size_t)c->vocab_size, L = (size_t)c->num_layers;
    if (c->wtype == JY_Q8_0 && (d % 32 || q % 32 || F % 32)) return -1;
    if (c->tied && c->wtype != JY_Q8_0) return -1; /* jieyu needs an f32 lm_head as [hidden][vocab] */
    const int t = c->wtype;

    /* arena plan */
    size_t off = 0;
    const size_t o_embed = off; off = align64(off + wbytes(t, V, d));
    const size_t o_lm = off; if (!c->tied) off = align64(off + wbytes(t, V, d));
    const size_t o_final = off; off = align64(off + d * 4);
    size_t* lo = (size_t*)calloc(L * L_NSLOT, sizeof(size_t));
    if (!lo) return -1;
    for (size_t l = 0; l < L; l++) {
        size_t* s = lo + l * L_NSLOT;
        s[L_RMS1] = off; off = align64(off + d * 4);
        s[L_WQ] = off; off = align64(off + wbytes(t, q, d));
        s[L_WK] = off; off = align64(off + wbytes(t, kv, d));
        s[L_WV] = off; off = align64(off + wbytes(t, kv, d));
        s[L_WO] = off; off = align64(off + wbytes(t, d, q));
        if (c->qkv_bias) {
            s[L_BQ] = off; off = align64(off + q * 4);
            s[L_BK] = off; off = align64(off + kv * 4);
            s[L_BV] = off; off = align64(off + kv * 4);
        }
        s[L_RMS2] = off; off = align64(off + d * 4);
        s[L_W1] = off; off = align64(off + wbytes(t, F, d));
        s[L_W2] = off; off = align64(off + wbytes(t, d, F));
        s[L_W3] = off; off = align64(off + wbytes(t, F, d));
    }
    jy_synth_model* m = (jy_synth_model*)calloc(1, sizeof(*m));
    jy_layer_weights* lw = (jy_layer_weights*)calloc(L, sizeof(*lw));
    void* arena = NULL;
    if (posix_memalign(&arena, 4096, off ? off : 64)) arena = NULL;
    if (!m || !lw || !arena) {
        free(m); free(lw); free(arena); free(lo);
        return -1;
    }
    uint8_t* A = (uint8_t*)arena;
    const uint64_t S = c->seed;
    const float sd = c->std;

    /* embedding rows are [vocab][hidden] for both types */
    fill_matrix(S, S_EMBED, sd, t, V, d, 1, A + o_embed);
    if (!c->tied) fill_matrix(S, S_LMHEAD, sd, t, V, d, 0, A + o_lm); /* f32: stored [hidden][vocab] */
    fill_norm(S, S_FINAL, sd, (float*)(A + o_final), d);
    for (size_t l = 0; l < L; l++) {
        const size_t* s = lo + l * L_NSLOT;
        jy_layer_weights* w = lw + l;
        fill_norm(S, layer_stream((int)l, L_RMS1), sd, (float*)(A + s[L_RMS1]), d);
        fill_matrix(S, layer_stream((int)l, L_WQ), sd, t, q, d, 0, A + s[L_WQ]);
        fill_matrix(S, layer_stream((int)l, L_WK), sd, t, kv, d, 0, A + s[L_WK]);
        fill_matrix(S, layer_stream((int)l, L_WV), sd, t, kv, d, 0, A + s[L_WV]);
        fill_matrix(S, layer_stream((int)l, L_WO), sd, t, d, q, 0, A + s[L_WO]);
        if (c->qkv_bias) {
            jysyn_normal_fill(S, layer_stream((int)l, L_BQ), sd, (float*)(A + s[L_BQ]), q);
            jysyn_normal_fill(S, layer_stream((int)l, L_BK), sd, (float*)(A + s[L_BK]), kv);
            jysyn_normal_fill(S, layer_stream((int)l, L_BV), sd, (float*)(A + s[L_BV]), kv);
            w->bq = (const float*)(A + s[L_BQ]);
            w->bk = (const float*)(A + s[L_BK]);
            w->bv = (const float*)(A + s[L_BV]);
        }
        fill_norm(S, layer_stream((int)l, L_RMS2), sd, (float*)(A + s[L_RMS2]), d);
        fill_matrix(S, layer_stream((int)l, L_W1), sd, t, F, d, 0, A + s[L_W1]);
        fill_matrix(S, layer_stream((int)l, L_W2), sd, t, d, F, 0, A + s[L_W2]);
        fill_matrix(S, layer_stream((int)l, L_W3), sd, t, F, d, 0, A + s[L_W3]);
        w->rms1_weight = (const float*)(A + s[L_RMS1]);
        w->rms2_weight = (const float*)(A + s[L_RMS2]);
        w->Wq.data = A + s[L_WQ]; w->Wq.type = t;
        w->Wk.data = A + s[L_WK]; w->Wk.type = t;
        w->Wv.data = A + s[L_WV]; w->Wv.type = t;
        w->Wo.data = A + s[L_WO]; w->Wo.type = t;
        w->W1.data = A + s[L_W1]; w->W1.type = t;
        w->W2.data = A + s[L_W2]; w->W2.type = t;
        w->W3.data = A + s[L_W3]; w->W3.type = t;
    }
    free(lo);

    jy_model_desc* D = &m->desc;
    D->num_layers = c->num_layers;
    D->hidden = c->hidden;
    D->num_heads = c->num_heads;
    D->num_kv_heads = c->num_kv_heads;
    D->head_dim = c->head_dim;
    D->intermediate = c->intermediate;
    D->vocab_size = c->vocab_size;
    D->rope_theta = (float)c->rope_theta;
    D->embed.data = A + o_embed; D->embed.type = t;
    D->lm_head.data = A + (c->tied ? o_embed : o_lm); D->lm_head.type = t;
    D->final_rms_weight = (const float*)(A + o_final);
    D->layers = lw;
    m->layers = lw;
    m->arena = arena;
    m->arena_bytes = off;
    m->weight_bytes = L * (wbytes(t, q, d) + 2 * wbytes(t, kv, d) + wbytes(t, d, q) + 3 * wbytes(t, F, d)) +
                      wbytes(t, V, d);
    *out = m;
    return 0;
}

void jysyn_free(jy_synth_model* m) {
    if (!m) return;
    free(m->arena);
    free(m->layers);
    free(m);
}
