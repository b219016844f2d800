// jy_runtime.cpp — host side of the MI355X decode path (C++17 over HIP).
//
// Owns device-resident models and KV caches and drives the per-token step:
// prefill (the prompt, seq > 1) launches the GEMM kernels directly; every later
// token replays one captured HIP graph whose kernels read the position from a
// device-side state word, so no host round trip is needed between tokens.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "jieyu_amd.h"
#include "jy_kernels.h"

using namespace jy;

// The workspace of jyhip_forward_cached_noalloc: a fixed array in every GPU's memory,
// held until the process ends.  In host code the name is only a stand-in for the
// symbol, never a device address.
static __device__ __align__(256) unsigned char scratch[JYHIP_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err;

struct Error {
    std::string msg;
};

void fail(const std::string& m) { throw Error{m}; }

void ck(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

#define CK(x) ck((x), #x)

template <class T>
T* dalloc(size_t n, bool zero = true) {
    void* p = nullptr;
    if (n == 0) n = 1;
    CK(hipMalloc(&p, n * sizeof(T)));
    if (zero) CK(hipMemset(p, 0, n * sizeof(T)));
    return (T*)p;
}

void dfree(void* p) {
    if (p) (void)hipFree(p);
}

// RoPETable::init (libs/date_libs/date.h:52-66): float arithmetic with the host
// libm, the same functions the reference calls, so the tables are identical.
void rope_table(int max_seq, int head_dim, float theta, std::vector<float>& c, std::vector<float>& s) {
    const int half = head_dim / 2;
    c.resize((size_t)max_seq * half);
    s.resize((size_t)max_seq * half);
    for (int i = 0; i < max_seq; i++)
        for (int j = 0; j < half; j++) {
            const float freq = 1.0f / powf(theta, 2.0f * (float)j / (float)head_dim);
            const float ang = (float)i * freq;
            c[(size_t)i * half + j] = cosf(ang);
            s[(size_t)i * half + j] = sinf(ang);
        }
}

size_t q8_bytes(size_t rows, size_t cols) { return rows * (cols / 32) * 34; }

// per device: the address of `scratch` on that device (hipGetSymbolAddress), the only
// form in which host code hands the array to kernels or copies
void* g_scratch[64] = {};

// per-device set-up, once per device and process, with that device current: kernel
// attributes (dynamic LDS limits) and the device address of `scratch`
void init_device_kernels(int device) {
    static bool done[64] = {};
    if (device < 0 || device >= 64) fail("device index out of range");
    if (done[device]) return;
    ck(kernels_init(), "kernel attributes");
    void* p = nullptr;
    ck(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) fail("hipGetSymbolAddress(scratch) returned NULL");
    g_scratch[device] = p;
    done[device] = true;
}

}  // namespace

// Models whose 2-D weights are not all Q8_0 or all f32 (f16, k-quants, or a mix,
// one type per matrix as jieyu's WMat allows) run each matrix on its own kernel.
constexpr int WT_MIXED = -1;

struct DevLayer {
    float* rms1 = nullptr;
    float* rms2 = nullptr;
    float* bqkv = nullptr;
    Q8Dev qkv, o, gu, down;                        // JY_Q8_0
    Q8MfmaDev mqkv, mo, mgu, mdown;                // their matrix-core GEMM copies (MFMA prefill mode)
    float *f_qkv = nullptr, *f_o = nullptr;        // JY_F32 [K][N] in 64-column panels of pieces
    float *f_w1 = nullptr, *f_w3 = nullptr, *f_w2 = nullptr;
    DevW w[7];                                     // WT_MIXED: Wq Wk Wv Wo W1 W2 W3
};

struct Workspace {
    int rows = 0;  // capacity in token rows
    float *X = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *g = nullptr, *u = nullptr, *h = nullptr;
    int8_t* q8 = nullptr;
    float* qsc = nullptr;
    float* scores = nullptr;
    size_t scores_n = 0;
    float* part = nullptr;  // split attention: per (query head, slice) o[hd], max, sum
    size_t part_n = 0;
    // matrix-core prompt GEMMs: the activations' fp16 high / low parts and row unscales
    _Float16 *ah = nullptr, *al = nullptr;
    float* aus = nullptr;
    size_t a_cap = 0;  // halves per part
    int a_rows = 0;    // rows of aus
    float* kp = nullptr;  // partial sums of the matrix-core GEMMs split over K
    size_t kp_n = 0;
    unsigned gen = 0;  // bumped whenever a buffer above is replaced: graphs captured before are stale
};

struct jyhip_model {
    int device = 0;
    int L = 0, H = 0, nh = 0, nkv = 0, hd = 0, F = 0, V = 0;
    int qd = 0, kvd = 0;
    int wtype = JY_Q8_0;
    int mode = JYHIP_MODE_EXACT;
    bool mfma_built = false;  // the layers' Q8MfmaDev copies exist
    bool bias = false;
    int max_seq = 0;
    float theta = 0.0f;
    float *cos_t = nullptr, *sin_t = nullptr;
    Q8Dev embed_q8, lm_q8;
    bool lm_shares_embed = false;
    float *embed_f32 = nullptr, *lm_f32 = nullptr;
    DevW embed_w, lm_w;  // WT_MIXED
    float* final_rms = nullptr;
    std::vector<DevLayer> layers;
    size_t weight_bytes = 0;
    double upload_ms = 0.0;
    hipStream_t stream = nullptr;
    Workspace ws;
    // the generation whose token ids and length the device buffers (ids, state) hold:
    // a session can step only while it is the latest one begun on its model
    const void* owner = nullptr;
    float* logits = nullptr;
    int* ids = nullptr;      // [max_seq + 1]
    int* state = nullptr;    // [0] = sequence length, [1] = stop flag
    int* eos = nullptr;      // [eos_cap]
    int eos_cap = 0;
    float* part_val = nullptr;  // lm_head argmax partials
    int* part_idx = nullptr;
    // the persistent decode kernel (Q8_0 models whose shapes it runs with one workgroup per CU)
    PLayer* pk_layers = nullptr;  // device [L]: each matrix's stream plan
    PMat pk_lm;
    unsigned* pk_flags = nullptr;  // barrier flags of the workgroups, then the attention slice counters
    size_t pk_flag_bytes = 0;
    int* pk_err = nullptr;         // set by the kernel when a barrier wait gave up
    size_t pk_lds = 0;
    std::vector<void*> owned;
};

struct jyhip_kv {
    KVDev dev;
    int current_len = 0;
    int device = 0;
};

struct jyhip_wmat {
    std::vector<DevW> copies;
    std::vector<void*> owned;
    int n = 0, k = 0;
    hipStream_t stream = nullptr;
};

struct jyhip_q8mat {
    int mode = JYHIP_MODE_EXACT;
    std::vector<Q8Dev> copies;
    std::vector<Q8MfmaDev> mcopies;  // the matrix-core GEMM's copies (built with JYHIP_MODE_MFMA_PREFILL)
    std::vector<void*> mowned;
    float* x = nullptr;
    float* y = nullptr;
    float* nw = nullptr;  // unit RMSNorm weights for the gate/up timing variant
    hipStream_t stream = nullptr;
    int next = 0;
};

namespace {

void* own(jyhip_model* m, void* p) {
    m->owned.push_back(p);
    return p;
}

Q8Dev q8_alloc(jyhip_model* m, int rows, int cols) {
    Q8Dev q = q8_shape(rows, cols);
    q.qs = (uint8_t*)own(m, dalloc<uint8_t>(q8_qs_bytes(rows, cols)));
    q.d = (uint16_t*)own(m, dalloc<uint8_t>(q8_d_bytes(rows, cols)));
    return q;
}

// host jieyu Q8_0 rows -> staging -> tiled rows [row_base + r*row_stride]
void q8_put(jyhip_model* m, uint8_t* staging, const void* src, int rows, int cols, const Q8Dev& dst, int row_base,
            int row_stride) {
    if (!src) fail("missing Q8_0 tensor");
    CK(hipMemcpy(staging, src, q8_bytes(rows, cols), hipMemcpyHostToDevice));
    launch_repack_q8(staging, rows, cols, dst, row_base, row_stride, m->stream);
    CK(hipGetLastError());
    CK(hipStreamSynchronize(m->stream));
}

float* f32_put(jyhip_model* m, const void* src, size_t n) {
    if (!src) fail("missing f32 tensor");
    float* d = (float*)own(m, dalloc<float>(n, false));
    CK(hipMemcpy(d, src, n * sizeof(float), hipMemcpyHostToDevice));
    return d;
}

void ensure_ws(jyhip_model* m, int rows) {
    Workspace& w = m->ws;
    if (w.rows >= rows) return;
    const unsigned gen = w.gen;
    for (void* p : {(void*)w.X, (void*)w.xn, (void*)w.qkv, (void*)w.att, (void*)w.g, (void*)w.u, (void*)w.h,
                    (void*)w.q8, (void*)w.qsc})
        dfree(p);
    float* const scores = w.scores;  // kept: sized by ensure_scores / ensure_part
    const size_t scores_n = w.scores_n;
    float* const part = w.part;
    const size_t part_n = w.part_n;
    const Workspace split = w;  // the MFMA split buffers are kept too (ensure_split)
    w = Workspace{};
    w.scores = scores;
    w.scores_n = scores_n;
    w.part = part;
    w.part_n = part_n;
    w.ah = split.ah;
    w.al = split.al;
    w.aus = split.aus;
    w.a_cap = split.a_cap;
    w.a_rows = split.a_rows;
    w.kp = split.kp;
    w.kp_n = split.kp_n;
    const size_t r = (size_t)rows;
    w.X = dalloc<float>(r * m->H);
    w.xn = dalloc<float>(r * m->H);
    w.qkv = dalloc<float>(r * (m->qd + 2 * m->kvd));
    w.att = dalloc<float>(r * m->qd);
    w.g = dalloc<float>(r * 2 * m->F);
    w.u = dalloc<float>(r * m->F);
    w.h = dalloc<float>(r * m->F);
    w.q8 = dalloc<int8_t>(r * m->qd);
    w.qsc = dalloc<float>(r * m->nh);
    w.rows = rows;
    w.gen = gen + 1;
}

void ensure_scores(jyhip_model* m, size_t n) {
    Workspace& w = m->ws;
    if (w.scores_n >= n) return;
    dfree(w.scores);
    w.scores = dalloc<float>(n, false);
    w.scores_n = n;
    w.gen++;
}

// the matrix-core GEMMs' split buffers: `halves` per part, `rows` unscales
void ensure_split(jyhip_model* m, size_t halves, int rows) {
    Workspace& w = m->ws;
    if (w.a_cap >= halves && w.a_rows >= rows) return;
    dfree(w.ah);
    dfree(w.al);
    dfree(w.aus);
    w.ah = w.al = nullptr;
    w.aus = nullptr;
    w.a_cap = 0;
    w.a_rows = 0;
    w.ah = reinterpret_cast<_Float16*>(dalloc<uint16_t>(halves, false));
    w.al = reinterpret_cast<_Float16*>(dalloc<uint16_t>(halves, false));
    w.aus = dalloc<float>((size_t)rows, false);
    w.a_cap = halves;
    w.a_rows = rows;
}

// the partial sums of the matrix-core GEMMs split over K (floats)
void ensure_kpart(jyhip_model* m, size_t n) {
    Workspace& w = m->ws;
    if (w.kp_n >= n) return;
    dfree(w.kp);
    w.kp = nullptr;
    w.kp_n = 0;
    w.kp = dalloc<float>(n, false);
    w.kp_n = n;
}

// a matrix's copy for the matrix-core GEMM (allocation recorded in `owned`)
Q8MfmaDev mfma_copy(std::vector<void*>& owned, const Q8Dev& W, hipStream_t st) {
    Q8MfmaDev M;
    M.rows = W.rows;
    M.cols = W.cols;
    M.nb = W.nb;
    M.nb4 = (W.nb + 3) / 4;
    M.tiles = (W.rows + 15) / 16;
    M.q = reinterpret_cast<int8_t*>(dalloc<uint8_t>((size_t)M.tiles * M.nb * 512, false));
    owned.push_back(M.q);
    M.d = dalloc<float>((size_t)M.tiles * M.nb4 * 64, false);
    owned.push_back(M.d);
    launch_mfma_repack(W, M, st);
    CK(hipGetLastError());
    return M;
}

// the layers' matrix-core copies, built once when a Q8_0 model first enables MFMA prefill
void build_mfma(jyhip_model* m) {
    if (m->mfma_built || m->wtype != JY_Q8_0) return;
    for (DevLayer& D : m->layers) {
        D.mqkv = mfma_copy(m->owned, D.qkv, m->stream);
        D.mo = mfma_copy(m->owned, D.o, m->stream);
        D.mgu = mfma_copy(m->owned, D.gu, m->stream);
        D.mdown = mfma_copy(m->owned, D.down, m->stream);
    }
    CK(hipStreamSynchronize(m->stream));
    m->mfma_built = true;
}

// whether a prompt pass runs its Q8_0 GEMMs on the matrix cores, and the split size it needs
bool use_mfma(const jyhip_model* m) {
    return m->wtype == JY_Q8_0 && (m->mode & JYHIP_MODE_MFMA_PREFILL) && m->mfma_built;
}
size_t mfma_split_halves(const jyhip_model* m, int seq) {
    return (size_t)mfma_rows_padded(seq) * std::max({m->H, m->qd, m->F});
}
// the partial floats a prompt pass of `seq` rows takes for its GEMMs split over K (every
// layer has the same shapes)
size_t mfma_kpart_need(const jyhip_model* m, int seq) {
    if (m->layers.empty() || !m->mfma_built) return 0;
    const DevLayer& D = m->layers[0];
    return std::max({gemm_q8_mfma_kpart_floats(D.mqkv, seq, D.bqkv ? EPI_BIAS : EPI_STORE),
                     gemm_q8_mfma_kpart_floats(D.mo, seq, EPI_RESID),
                     gemm_q8_mfma_kpart_floats(D.mdown, seq, EPI_RESID)});
}

void ensure_part(jyhip_model* m, size_t n) {
    Workspace& w = m->ws;
    if (w.part_n >= n) return;
    dfree(w.part);
    w.part = dalloc<float>(n, false);
    w.part_n = n;
    w.gen++;
}

// a decode Q8_0 matvec in the model's mode: the reference's 32-lane order, or the split dot;
// with JYHIP_MODE_SPLIT_MV the larger matrices keep the 32-lane order with the RMSNorm
// applied after the dot (linearity)
void q8_matvec(const jyhip_model* m, const Q8Dev& W, const float* x, const float* norm_w, float* out, Epi epi,
               const MvArgs& a, hipStream_t st) {
    if ((m->mode & JYHIP_MODE_SPLIT_MV) && W.rows < JYHIP_SPLIT_MV_ROWS)
        launch_matvec_q8_split(W, x, norm_w, out, epi, a, st);
    else
        launch_matvec_q8(W, x, norm_w, out, epi, a, st, (m->mode & JYHIP_MODE_SPLIT_MV) != 0);
}

// the decode attention runs split across workgroups (flash-decoding)
bool split_attention(const jyhip_model* m) {
    return (m->mode & JYHIP_MODE_SPLIT_ATTN) && m->wtype == JY_Q8_0 && attn_split_supported(m->nh, m->nkv, m->hd);
}

// the longest sequence whose decode step takes the short-context attention: the split mode's
// whole-range kernel, or the exact mode's one-kernel form
int short_keys(const jyhip_model* m) { return split_attention(m) ? att_whole_keys() : att_short_keys(); }

// slice partials (floats) a decode step attending up to max_keys keys takes: the separate
// kernels' slice count or the persistent kernel's, whichever is larger (either may run)
size_t part_need(const jyhip_model* m, int max_keys) {
    if (!split_attention(m)) return 0;
    const int ns = std::max(attn_split_slices(max_keys), persist_slices(m->nkv, max_keys));
    return attn_split_part_floats(m->nh, m->hd, ns);
}

// the decode step runs as the persistent kernel: asked for, its shapes supported, and the
// mode has both split forms it is built from
bool use_persist(const jyhip_model* m) {
    return m->pk_layers && (m->mode & JYHIP_MODE_PERSIST) && (m->mode & JYHIP_MODE_SPLIT_MV) &&
           (m->mode & JYHIP_MODE_SPLIT_ATTN);
}

// one decode row (position state[0]-1, or pos0 without state) of every layer in the
// persistent kernel over workspace w; with head, also the final norm, lm_head and the greedy
// pick; with layer_x (device [L][H]) X after every layer
void launch_persist(jyhip_model* m, Workspace& w, const KVDev& kv, const int* state, int pos0, int max_keys,
                    float* layer_x, bool head, int neos) {
    PersistArgs A;
    A.layers = m->pk_layers;
    A.L = m->L;
    A.H = m->H;
    A.F = m->F;
    A.lm = m->pk_lm;
    A.final_rms = m->final_rms;
    A.cos_t = m->cos_t;
    A.sin_t = m->sin_t;
    A.att.fused = true;
    A.att.qkv = w.qkv;
    A.att.nrows = 1;
    A.att.row0 = 0;
    A.att.start_pos = pos0;
    A.att.state = state;
    A.att.nh = m->nh;
    A.att.nkv = m->nkv;
    A.att.hd = m->hd;
    A.att.kv = kv;
    A.att.max_keys = max_keys;
    A.att.out = w.att;
    A.X = w.X;
    A.qkv = w.qkv;
    A.h = w.h;
    A.part = w.part;
    A.ns = persist_slices(m->nkv, max_keys);
    A.flags = m->pk_flags;
    A.acnt = m->pk_flags + persist_workgroups();
    A.err = m->pk_err;
    A.layer_x = layer_x;
    A.head = head ? 1 : 0;
    if (head) {
        A.logits = m->logits;
        A.part_val = m->part_val;
        A.part_idx = m->part_idx;
        A.ids = m->ids;
        A.mstate = m->state;
        A.eos = m->eos;
        A.neos = neos;
    }
    launch_zero_fill(m->pk_flags, m->pk_flag_bytes, m->stream);  // flags and counters start at zero
    launch_decode_persist(A, m->pk_lds, m->stream);
}

// after the stream is synchronised: a persistent step whose barrier wait gave up is an error
void check_persist(jyhip_model* m) {
    if (!m->pk_err) return;
    int e = 0;
    CK(hipMemcpy(&e, m->pk_err, sizeof(int), hipMemcpyDeviceToHost));
    if (e) {
        launch_zero_fill(m->pk_err, 16, m->stream);
        CK(hipStreamSynchronize(m->stream));
        fail("decode step: the persistent kernel's workgroups did not all meet at a barrier (not all resident?)");
    }
}

bool known_type(int t) {
    return t == JY_F32 || t == JY_F16 || t == JY_Q8_0 || t == JY_Q4_K || t == JY_Q5_K || t == JY_Q6_K;
}

int block_of(int t) { return t == JY_Q8_0 ? 32 : (t == JY_Q4_K || t == JY_Q5_K || t == JY_Q6_K) ? 256 : 1; }

// the path a model runs: JY_Q8_0 (every matrix Q8_0), JY_F32 (every matrix f32), else WT_MIXED
int check_desc(const jy_model_desc* d) {
    if (!d) fail("model description is NULL");
    if (d->num_layers <= 0 || d->hidden <= 0 || d->num_heads <= 0 || d->num_kv_heads <= 0 || d->head_dim <= 0 ||
        d->intermediate <= 0 || d->vocab_size <= 0)
        fail("model hyper-parameters must be positive");
    if (d->num_heads % d->num_kv_heads) fail("num_heads must be a multiple of num_kv_heads");
    if (d->head_dim % 4 || d->head_dim > 256) fail("head_dim must be a multiple of 4 and at most 256");
    if (!d->layers || !d->final_rms_weight) fail("layers / final norm missing");
    const int H = d->hidden, qd = d->num_heads * d->head_dim, F = d->intermediate;
    int first = d->layers[0].Wq.type;
    bool same = true;
    auto check = [&](const jy_wmat& x, int in, const char* what) {
        if (!x.data) fail(std::string(what) + " missing");
        if (!known_type(x.type)) fail(std::string("unsupported weight type for ") + what);
        if (in % block_of(x.type))
            fail(std::string(what) + ": input width " + std::to_string(in) + " is not a multiple of its block size");
        same = same && x.type == first;
    };
    for (int l = 0; l < d->num_layers; l++) {
        const jy_layer_weights& w = d->layers[l];
        check(w.Wq, H, "Wq");
        check(w.Wk, H, "Wk");
        check(w.Wv, H, "Wv");
        check(w.Wo, qd, "Wo");
        check(w.W1, H, "W1");
        check(w.W2, F, "W2");
        check(w.W3, H, "W3");
        if (!w.rms1_weight || !w.rms2_weight) fail("norm weights missing");
        if ((w.bq != nullptr) != (d->layers[0].bq != nullptr)) fail("q/k/v biases must be on every layer or none");
        if ((w.bq == nullptr) != (w.bk == nullptr) || (w.bq == nullptr) != (w.bv == nullptr))
            fail("q/k/v biases must come together");
    }
    check(d->embed, H, "embedding");
    // a quantized lm_head is [vocab][hidden] (input width hidden); f32 / f16 is [hidden][vocab]
    check(d->lm_head, H, "lm_head");
    if (same && (first == JY_Q8_0 || first == JY_F32)) {
        if (first == JY_Q8_0 && (H % 32 || F % 32 || qd % 32))
            fail("Q8_0 needs hidden, intermediate and q_dim divisible by 32");
        return first;
    }
    return WT_MIXED;
}

size_t wbytes(int type, size_t out, size_t in) {
    switch (type) {
        case JY_F32: return out * in * 4;
        case JY_F16: return out * in * 2;
        case JY_Q8_0: return out * (in / 32) * 34;
        case JY_Q4_K: return out * (in / 256) * 144;
        case JY_Q5_K: return out * (in / 256) * 176;
        default: return out * (in / 256) * 210;
    }
}

// A dense [K][N] matrix (jieyu's [in][out]) as ceil(N/64) panels, each holding 64
// columns as 16-byte pieces [ceil(K/per)][64][per] (per = 16 / element size): piece
// (kb, c) is column c's elements kb*per .. kb*per + per - 1.  Columns past N and
// rows past K are zero.  The decode matvec's workgroup for panel p then streams one
// contiguous run, and lane c of its chain wave reads whole pieces of its column.
template <typename E>
void dense_pack(const E* s, int K, int N, E* h) {
    const int per = 16 / (int)sizeof(E), nkb = (K + per - 1) / per;
    for (int k = 0; k < K; k++) {
        const E* row = s + (size_t)k * N;
        for (int j = 0; j < N; j++) h[(((size_t)(j / 64) * nkb + k / per) * 64 + j % 64) * per + k % per] = row[j];
    }
}

void* dense_put(jyhip_model* m, const void* src, int K, int N, int es) {
    if (!src) fail("missing dense tensor");
    const int per = 16 / es, nkb = (K + per - 1) / per, np = (N + 63) / 64;
    std::vector<uint8_t> h((size_t)np * nkb * 64 * 16, 0);
    if (es == 4)
        dense_pack(static_cast<const uint32_t*>(src), K, N, reinterpret_cast<uint32_t*>(h.data()));
    else
        dense_pack(static_cast<const uint16_t*>(src), K, N, reinterpret_cast<uint16_t*>(h.data()));
    void* d = own(m, dalloc<uint8_t>(h.size(), false));
    CK(hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice));
    return d;
}

// one matrix of out x in weights (quantized [out][in]; f32 / f16 [in][out], in 64-column
// panels unless `panels` is false: the embedding table keeps its [vocab][hidden] rows)
DevW put_w(jyhip_model* m, uint8_t* staging, const jy_wmat& src, int out, int in, bool panels = true) {
    DevW w;
    w.type = src.type;
    w.in = in;
    w.out = out;
    const size_t nb = wbytes(src.type, out, in);
    if (src.type == JY_F32 || src.type == JY_F16) {
        if (panels) {
            w.dense = dense_put(m, src.data, in, out, src.type == JY_F32 ? 4 : 2);
        } else {
            void* p = own(m, dalloc<uint8_t>(nb, false));
            CK(hipMemcpy(p, src.data, nb, hipMemcpyHostToDevice));
            w.dense = p;
        }
    } else if (src.type == JY_Q8_0) {
        w.q8 = q8_alloc(m, out, in);
        q8_put(m, staging, src.data, out, in, w.q8, 0, 1);
    } else {
        w.kq = kq_shape(src.type, out, in);
        w.kq.nib = (uint8_t*)own(m, dalloc<uint8_t>(kq_bytes(w.kq, 0)));
        if (kq_bytes(w.kq, 1)) w.kq.hi = (uint8_t*)own(m, dalloc<uint8_t>(kq_bytes(w.kq, 1)));
        w.kq.hdr = (uint8_t*)own(m, dalloc<uint8_t>(kq_bytes(w.kq, 2)));
        w.kq.dm = (uint32_t*)own(m, dalloc<uint8_t>(kq_bytes(w.kq, 3)));
        CK(hipMemcpy(staging, src.data, nb, hipMemcpyHostToDevice));
        launch_repack_kq(staging, w.kq, m->stream);
        CK(hipGetLastError());
        CK(hipStreamSynchronize(m->stream));
    }
    return w;
}

void upload_mixed(jyhip_model* m, const jy_model_desc* d) {
    const int H = m->H, qd = m->qd, kvd = m->kvd, F = m->F, V = m->V;
    // the x vector of a k-quant decode matvec is staged in LDS
    for (int in : {H, qd, F})
        if (mv_kq_lds_bytes(in) > matvec_lds_limit() || matvec_lds_bytes(in, false) > matvec_lds_limit())
            fail("hidden / q_dim / intermediate too large for the decode matvec's LDS staging");
    size_t stage = std::max(wbytes(d->embed.type, V, H), wbytes(d->lm_head.type, V, H));
    for (int l = 0; l < m->L; l++) {
        const jy_layer_weights& w = d->layers[l];
        stage = std::max({stage, wbytes(w.Wq.type, qd, H), wbytes(w.Wk.type, kvd, H), wbytes(w.Wv.type, kvd, H),
                          wbytes(w.Wo.type, H, qd), wbytes(w.W1.type, F, H), wbytes(w.W2.type, H, F),
                          wbytes(w.W3.type, F, H)});
    }
    uint8_t* staging = dalloc<uint8_t>(stage, false);
    size_t total = 0;
    try {
        m->embed_w = put_w(m, staging, d->embed, V, H, false);
        total += wbytes(d->embed.type, V, H);
        const bool dense_lm = d->lm_head.type == JY_F32 || d->lm_head.type == JY_F16;
        if (d->lm_head.data == d->embed.data && d->lm_head.type == d->embed.type && !dense_lm) {
            m->lm_w = m->embed_w;  // tied (load_weights.h:143-144)
        } else {
            m->lm_w = put_w(m, staging, d->lm_head, V, H);
            total += wbytes(d->lm_head.type, V, H);
        }
        for (int l = 0; l < m->L; l++) {
            const jy_layer_weights& w = d->layers[l];
            DevLayer& D = m->layers[l];
            D.rms1 = f32_put(m, w.rms1_weight, H);
            D.rms2 = f32_put(m, w.rms2_weight, H);
            const jy_wmat* src[7] = {&w.Wq, &w.Wk, &w.Wv, &w.Wo, &w.W1, &w.W2, &w.W3};
            const int outs[7] = {qd, kvd, kvd, H, F, H, F}, ins[7] = {H, H, H, qd, H, F, H};
            for (int i = 0; i < 7; i++) {
                D.w[i] = put_w(m, staging, *src[i], outs[i], ins[i]);
                total += wbytes(src[i]->type, outs[i], ins[i]);
            }
        }
    } catch (...) {
        dfree(staging);
        throw;
    }
    dfree(staging);
    m->weight_bytes = total;
}

PMat pmat(const Q8Dev& q, int nwg) {
    PMat p;
    p.qs = q.qs;
    p.d = q.d;
    p.rows = q.rows;
    p.cols = q.cols;
    p.nch = q.nch;
    p.nchp = q.nchp;
    p.nbp = q.nbp;
    persist_plan(p, nwg);
    return p;
}

// the persistent decode kernel's per-model state: every matrix's stream plan on the device,
// the barrier flags and the error word; left unset (the separate kernels run instead) for
// shapes it does not take or when one workgroup per CU would not stay resident
void build_persist(jyhip_model* m) {
    if (m->wtype != JY_Q8_0 || !persist_supported(m->nh, m->nkv, m->hd)) return;
    const int nwg = persist_workgroups();
    std::vector<PLayer> h(m->L);
    int max_nbp = 0;
    for (int l = 0; l < m->L; l++) {
        const DevLayer& D = m->layers[l];
        h[l].qkv = pmat(D.qkv, nwg);
        h[l].o = pmat(D.o, nwg);
        h[l].gu = pmat(D.gu, nwg);
        h[l].down = pmat(D.down, nwg);
        h[l].rms1 = D.rms1;
        h[l].rms2 = D.rms2;
        h[l].bqkv = D.bqkv;
        max_nbp = std::max({max_nbp, D.qkv.nbp, D.o.nbp, D.gu.nbp, D.down.nbp});
    }
    PMat lm = pmat(m->lm_q8, nwg);
    max_nbp = std::max(max_nbp, lm.nbp);
    const size_t lds = persist_lds_bytes(max_nbp, m->hd);
    if (!persist_resident(m->hd, lds)) return;
    m->pk_layers = (PLayer*)own(m, dalloc<PLayer>(m->L));
    CK(hipMemcpy(m->pk_layers, h.data(), sizeof(PLayer) * m->L, hipMemcpyHostToDevice));
    m->pk_lm = lm;
    m->pk_flag_bytes = (size_t)(nwg + m->nkv + 3) / 4 * 16;
    m->pk_flags = (unsigned*)own(m, dalloc<uint8_t>(m->pk_flag_bytes));
    m->pk_err = (int*)own(m, dalloc<int>(4));
    m->pk_lds = lds;
}

void upload(jyhip_model* m, const jy_model_desc* d, int max_seq, int wtype) {
    m->L = d->num_layers;
    m->H = d->hidden;
    m->nh = d->num_heads;
    m->nkv = d->num_kv_heads;
    m->hd = d->head_dim;
    m->F = d->intermediate;
    m->V = d->vocab_size;
    m->qd = m->nh * m->hd;
    m->kvd = m->nkv * m->hd;
    m->wtype = wtype;
    m->bias = d->layers[0].bq != nullptr;
    m->max_seq = max_seq;
    m->theta = d->rope_theta;
    CK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));

    std::vector<float> c, s;
    rope_table(max_seq, m->hd, m->theta, c, s);
    m->cos_t = f32_put(m, c.data(), c.size());
    m->sin_t = f32_put(m, s.data(), s.size());
    m->final_rms = f32_put(m, d->final_rms_weight, m->H);

    const int H = m->H, qd = m->qd, kvd = m->kvd, F = m->F, V = m->V;
    m->layers.resize(m->L);
    if (m->wtype == WT_MIXED) {
        upload_mixed(m, d);
    } else if (m->wtype == JY_Q8_0) {
        // the decode matvec stages its whole input vector in LDS (with the norm weights
        // where it normalises): hidden for QKV / gate-up / lm_head, q_dim for O, F for down
        if (matvec_lds_bytes(H, true) > matvec_lds_limit() || matvec_lds_bytes(qd, false) > matvec_lds_limit() ||
            matvec_lds_bytes(F, false) > matvec_lds_limit())
            fail("hidden / q_dim / intermediate too large for the decode matvec's LDS staging");
        size_t stage = q8_bytes(V, H);
        stage = std::max(stage, q8_bytes(F, H));
        stage = std::max(stage, q8_bytes(H, F));
        stage = std::max(stage, q8_bytes(qd, H));
        uint8_t* staging = dalloc<uint8_t>(stage, false);
        try {
            m->embed_q8 = q8_alloc(m, V, H);
            q8_put(m, staging, d->embed.data, V, H, m->embed_q8, 0, 1);
            m->lm_shares_embed = d->lm_head.data == d->embed.data;
            if (m->lm_shares_embed) {
                m->lm_q8 = m->embed_q8;
            } else {
                m->lm_q8 = q8_alloc(m, V, H);
                q8_put(m, staging, d->lm_head.data, V, H, m->lm_q8, 0, 1);
            }
            for (int l = 0; l < m->L; l++) {
                const jy_layer_weights& w = d->layers[l];
                DevLayer& D = m->layers[l];
                D.rms1 = f32_put(m, w.rms1_weight, H);
                D.rms2 = f32_put(m, w.rms2_weight, H);
                D.qkv = q8_alloc(m, qd + 2 * kvd, H);
                q8_put(m, staging, w.Wq.data, qd, H, D.qkv, 0, 1);
                q8_put(m, staging, w.Wk.data, kvd, H, D.qkv, qd, 1);
                q8_put(m, staging, w.Wv.data, kvd, H, D.qkv, qd + kvd, 1);
                D.o = q8_alloc(m, H, qd);
                q8_put(m, staging, w.Wo.data, H, qd, D.o, 0, 1);
                D.gu = q8_alloc(m, 2 * F, H);  // gate row i -> 2i, up row i -> 2i+1
                q8_put(m, staging, w.W1.data, F, H, D.gu, 0, 2);
                q8_put(m, staging, w.W3.data, F, H, D.gu, 1, 2);
                D.down = q8_alloc(m, H, F);
                q8_put(m, staging, w.W2.data, H, F, D.down, 0, 1);
            }
        } catch (...) {
            dfree(staging);
            throw;
        }
        dfree(staging);
        m->weight_bytes = (size_t)m->L * (q8_bytes(qd + 2 * kvd, H) + q8_bytes(H, qd) + q8_bytes(2 * F, H) +
                                          q8_bytes(H, F)) +
                          q8_bytes(V, H);
    } else {
        m->embed_f32 = f32_put(m, d->embed.data, (size_t)V * H);
        m->lm_f32 = (float*)dense_put(m, d->lm_head.data, H, V, 4);  // [hidden][vocab]
        const size_t NQ = (size_t)qd + 2 * kvd;
        for (int l = 0; l < m->L; l++) {
            const jy_layer_weights& w = d->layers[l];
            DevLayer& D = m->layers[l];
            D.rms1 = f32_put(m, w.rms1_weight, H);
            D.rms2 = f32_put(m, w.rms2_weight, H);
            {
                std::vector<float> qkv((size_t)H * NQ);  // [H][qd | kvd | kvd]
                const float* parts[3] = {static_cast<const float*>(w.Wq.data), static_cast<const float*>(w.Wk.data),
                                         static_cast<const float*>(w.Wv.data)};
                const int widths[3] = {qd, kvd, kvd};
                for (int k = 0; k < H; k++)
                    for (int i = 0, c = 0; i < 3; c += widths[i++])
                        memcpy(&qkv[(size_t)k * NQ + c], parts[i] + (size_t)k * widths[i], (size_t)widths[i] * 4);
                D.f_qkv = (float*)dense_put(m, qkv.data(), H, NQ, 4);
            }
            D.f_o = (float*)dense_put(m, w.Wo.data, qd, H, 4);
            D.f_w1 = (float*)dense_put(m, w.W1.data, H, F, 4);
            D.f_w3 = (float*)dense_put(m, w.W3.data, H, F, 4);
            D.f_w2 = (float*)dense_put(m, w.W2.data, F, H, 4);
        }
        m->weight_bytes = ((size_t)m->L * ((size_t)H * NQ + (size_t)qd * H + 3 * (size_t)H * F) + (size_t)H * V) * 4;
    }
    if (m->bias)
        for (int l = 0; l < m->L; l++) {
            const jy_layer_weights& w = d->layers[l];
            DevLayer& D = m->layers[l];
            D.bqkv = (float*)own(m, dalloc<float>((size_t)qd + 2 * kvd, false));
            CK(hipMemcpy(D.bqkv, w.bq, (size_t)qd * 4, hipMemcpyHostToDevice));
            CK(hipMemcpy(D.bqkv + qd, w.bk, (size_t)kvd * 4, hipMemcpyHostToDevice));
            CK(hipMemcpy(D.bqkv + qd + kvd, w.bv, (size_t)kvd * 4, hipMemcpyHostToDevice));
        }
    build_persist(m);
    m->logits = (float*)own(m, dalloc<float>(V));
    m->ids = (int*)own(m, dalloc<int>((size_t)max_seq + 1));
    m->state = (int*)own(m, dalloc<int>(4));
    m->eos_cap = 64;
    m->eos = (int*)own(m, dalloc<int>(m->eos_cap));
    // one partial maximum per lm_head workgroup of any of the decode forms
    const int np = std::max({argmax_partials(V), split_argmax_partials(V), persist_workgroups()});
    m->part_val = (float*)own(m, dalloc<float>(np));
    m->part_idx = (int*)own(m, dalloc<int>(np));
}

void release(jyhip_model* m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (void* p : m->owned) dfree(p);
    Workspace& w = m->ws;
    for (void* p : {(void*)w.X, (void*)w.xn, (void*)w.qkv, (void*)w.att, (void*)w.g, (void*)w.u, (void*)w.h,
                    (void*)w.q8, (void*)w.qsc, (void*)w.scores, (void*)w.part, (void*)w.ah, (void*)w.al,
                    (void*)w.aus, (void*)w.kp})
        dfree(p);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

// ---------------------------------------------------------------- the step

// transformer_layer x L (libs/model_libs/transformer_layer.h:10-90) for one token
// in ws.X at position state[0]-1 (state != null) or pos0: the m == 1 path of every
// matmul (matmul_q.h:139-144).  Q8_0: six kernels per layer (RMSNorm + QKV + RoPE,
// the two attention kernels with K/V packing, O + residual, RMSNorm + gate/up +
// SwiGLU, down + residual).
void run_decode_layers(jyhip_model* m, Workspace& w, const KVDev& kv, const int* state, int pos0,
                       float* layer_out_host, int max_keys, bool short_ctx = false) {
    hipStream_t st = m->stream;
    if (use_persist(m)) {
        float* lx = nullptr;
        if (layer_out_host) lx = dalloc<float>((size_t)m->L * m->H, false);
        try {
            launch_persist(m, w, kv, state, pos0, max_keys, lx, false, 0);
            CK(hipGetLastError());
            if (lx) {
                CK(hipMemcpyAsync(layer_out_host, lx, sizeof(float) * m->L * m->H, hipMemcpyDeviceToHost, st));
                CK(hipStreamSynchronize(st));
            }
        } catch (...) {
            if (lx) {
                (void)hipStreamSynchronize(st);
                dfree(lx);
            }
            throw;
        }
        if (lx) {
            dfree(lx);
            check_persist(m);
        }
        return;
    }
    const int H = m->H, NQ = m->qd + 2 * m->kvd, F = m->F;
    AttnArgs at;
    at.nrows = 1;
    at.start_pos = pos0;
    at.state = state;
    at.short_ctx = short_ctx;
    at.nh = m->nh;
    at.nkv = m->nkv;
    at.hd = m->hd;
    at.kv = kv;
    at.scratch = w.scores;
    at.max_keys = max_keys;
    at.out = w.att;
    for (int l = 0; l < m->L; l++) {
        const DevLayer& D = m->layers[l];
        at.layer = l;
        if (m->wtype == JY_Q8_0) {
            MvArgs qa;
            qa.aux = D.bqkv;
            qa.state = state;
            qa.pos0 = pos0;
            qa.cos_t = m->cos_t;
            qa.sin_t = m->sin_t;
            qa.nh = m->nh;
            qa.nkv = m->nkv;
            qa.hd = m->hd;
            q8_matvec(m, D.qkv, w.X, D.rms1, w.qkv, EPI_ROPE, qa, st);
            at.fused = true;
            at.qkv = w.qkv;
            if (split_attention(m) && (state ? short_ctx : pos0 + 1 <= att_whole_keys()))
                launch_attention_whole(at, st);
            else if (split_attention(m))
                launch_attention_split(at, w.part, attn_split_slices(max_keys), st);
            else
                launch_attention(at, st);
            const MvArgs none;
            q8_matvec(m, D.o, w.att, nullptr, w.X, EPI_RESID, none, st);
            q8_matvec(m, D.gu, w.X, D.rms2, w.h, EPI_SWIGLU, none, st);
            q8_matvec(m, D.down, w.h, nullptr, w.X, EPI_RESID, none, st);
        } else if (m->wtype == WT_MIXED) {
            // one kernel per matrix, each in its own type's order
            const int qd = m->qd, kvd = m->kvd;
            const Epi qe = D.bqkv ? EPI_BIAS : EPI_STORE;
            launch_rmsnorm(w.X, w.xn, D.rms1, H, 1, st);
            launch_mv(D.w[0], w.xn, w.qkv, qe, D.bqkv, st);
            launch_mv(D.w[1], w.xn, w.qkv + qd, qe, D.bqkv ? D.bqkv + qd : nullptr, st);
            launch_mv(D.w[2], w.xn, w.qkv + qd + kvd, qe, D.bqkv ? D.bqkv + qd + kvd : nullptr, st);
            launch_rope_pack(w.qkv, 1, pos0, state, m->nh, m->nkv, m->hd, m->cos_t, m->sin_t, kv, l, w.q8, w.qsc, st);
            at.fused = false;
            at.q8 = w.q8;
            at.qsc = w.qsc;
            at.row0 = 0;
            launch_attention(at, st);
            launch_mv(D.w[3], w.att, w.X, EPI_RESID, nullptr, st);
            launch_rmsnorm(w.X, w.xn, D.rms2, H, 1, st);
            launch_mv(D.w[4], w.xn, w.g, EPI_STORE, nullptr, st);
            launch_mv(D.w[6], w.xn, w.u, EPI_STORE, nullptr, st);
            launch_silu_mul(w.g, w.u, 0, 1, F, w.h, st);
            launch_mv(D.w[5], w.h, w.X, EPI_RESID, nullptr, st);
        } else {
            launch_rmsnorm(w.X, w.xn, D.rms1, H, 1, st);
            launch_matvec_f32(D.f_qkv, H, NQ, w.xn, w.qkv, D.bqkv, D.bqkv ? EPI_BIAS : EPI_STORE, st);
            launch_rope_pack(w.qkv, 1, pos0, state, m->nh, m->nkv, m->hd, m->cos_t, m->sin_t, kv, l, w.q8, w.qsc, st);
            at.fused = false;
            at.q8 = w.q8;
            at.qsc = w.qsc;
            at.row0 = 0;
            launch_attention(at, st);
            launch_matvec_f32(D.f_o, m->qd, H, w.att, w.X, nullptr, EPI_RESID, st);
            launch_rmsnorm(w.X, w.xn, D.rms2, H, 1, st);
            launch_matvec_f32(D.f_w1, H, F, w.xn, w.g, nullptr, EPI_STORE, st);
            launch_matvec_f32(D.f_w3, H, F, w.xn, w.h, w.g, EPI_SWIGLU, st);  // h = silu(gate) * up
            launch_matvec_f32(D.f_w2, F, H, w.h, w.X, nullptr, EPI_RESID, st);
        }
        if (layer_out_host) {
            CK(hipMemcpyAsync(layer_out_host + (size_t)l * H, w.X, sizeof(float) * H, hipMemcpyDeviceToHost, st));
            CK(hipStreamSynchronize(st));
        }
    }
    CK(hipGetLastError());
}

// the prompt (seq > 1): the generic m > 1 matmul path (matmul_q.h:145-161) as tiled
// GEMMs, RoPE + K/V packing of every row before attention.
void run_prefill_layers(jyhip_model* m, Workspace& w, const KVDev& kv, int seq, int start_pos,
                        float* layer_out_host, int max_keys) {
    hipStream_t st = m->stream;
    const bool q8 = m->wtype == JY_Q8_0, mixed = m->wtype == WT_MIXED;
    const int H = m->H, NQ = m->qd + 2 * m->kvd, F = m->F;
    // attention rows per launch keep the HBM score scratch within its allocation
    const size_t per_row = (size_t)m->nh * max_keys;
    const int chunk = (int)std::max<size_t>(1, std::min<size_t>(seq, w.scores_n / per_row));
    AttnArgs at;
    at.fused = false;
    at.q8 = w.q8;
    at.qsc = w.qsc;
    at.start_pos = start_pos;
    at.nh = m->nh;
    at.nkv = m->nkv;
    at.hd = m->hd;
    at.kv = kv;
    at.scratch = w.scores;
    at.max_keys = max_keys;
    at.out = w.att;
    // Q8_0 GEMMs: the exact tiles, or (MFMA prefill mode) the activations split into fp16
    // high / low parts and the matrix-core kernel
    const bool mf = q8 && use_mfma(m);
    // attention of the prompt rows: the tolerance mode's split form (one workgroup per kv
    // head and row) or the exact kernels over chunks of rows
    const bool split_rows = (m->mode & JYHIP_MODE_SPLIT_ATTN) && attn_split_supported(m->nh, m->nkv, m->hd);
    const int mp = mfma_rows_padded(seq);
    if (mf && (w.a_cap < mfma_split_halves(m, seq) || w.a_rows < mp)) {
        if (&w != &m->ws) fail("prefill: the workspace has no room for the matrix-core split buffers");
        ensure_split(m, mfma_split_halves(m, seq), mp);
    }
    if (mf && w.kp_n < mfma_kpart_need(m, seq)) {
        if (&w != &m->ws) fail("prefill: the workspace has no room for the matrix-core partial sums");
        ensure_kpart(m, mfma_kpart_need(m, seq));
    }
    // A matrix-core GEMM split over K may leave its sum to the next kernel (`defer`): the
    // QKV product's to rope_pack, a residual product's (O, down) to the next RMSNorm + split,
    // which adds the partials into X.  pending_x counts the partials a residual product left
    // in w.kp; resolve_x adds them where no such kernel follows (a layer's output copied out,
    // the last layer).
    const bool fuse_x = mf && mfma_norm_split_takes_parts(H);
    int pending_x = 0;
    auto resolve_x = [&]() {
        if (pending_x > 1) launch_gemm_ksum(w.kp, pending_x, seq, H, w.X, H, nullptr, EPI_RESID, st);
        pending_x = 0;
    };
    auto gemm_q8 = [&](const Q8Dev& W, const Q8MfmaDev& M, const float* A, float* Cm, const float* aux, Epi epi,
                       bool defer = false) {
        if (mf) {
            launch_mfma_split(A, seq, mp, W.cols, w.ah, w.al, w.aus, st);
            return launch_gemm_q8_mfma(M, seq, w.ah, w.al, w.aus, Cm, W.rows, aux, epi, st, w.kp, w.kp_n, defer);
        }
        launch_gemm_q8(W, seq, A, Cm, aux, epi, st);
        return 0;
    };
    // matrix-core form of RMSNorm + GEMM: the norm and the activation split in one kernel
    // (xn is not written; X first takes the partials a residual product left); `ldc` the
    // output row stride
    auto norm_gemm_q8 = [&](const Q8MfmaDev& M, const float* nw, float* Cm, int ldc, const float* aux, Epi epi,
                            bool defer = false) {
        launch_mfma_norm_split(w.X, seq, mp, H, nw, w.ah, w.al, w.aus, st, w.kp, pending_x);
        pending_x = 0;
        return launch_gemm_q8_mfma(M, seq, w.ah, w.al, w.aus, Cm, ldc, aux, epi, st, w.kp, w.kp_n, defer);
    };
    for (int l = 0; l < m->L; l++) {
        const DevLayer& D = m->layers[l];
        if (!mf) launch_rmsnorm(w.X, w.xn, D.rms1, H, seq, st);
        const Epi qkv_epi = D.bqkv ? EPI_BIAS : EPI_STORE;
        int pending_qkv = 0;  // partials of the QKV product, summed by rope_pack
        if (mixed) {
            const int qd = m->qd, kvd = m->kvd;
            launch_gemm(D.w[0], seq, w.xn, w.qkv, NQ, D.bqkv, qkv_epi, st);
            launch_gemm(D.w[1], seq, w.xn, w.qkv + qd, NQ, D.bqkv ? D.bqkv + qd : nullptr, qkv_epi, st);
            launch_gemm(D.w[2], seq, w.xn, w.qkv + qd + kvd, NQ, D.bqkv ? D.bqkv + qd + kvd : nullptr, qkv_epi, st);
        } else if (mf) {
            pending_qkv = norm_gemm_q8(D.mqkv, D.rms1, w.qkv, D.qkv.rows, D.bqkv, qkv_epi, true);
        } else if (q8) {
            gemm_q8(D.qkv, D.mqkv, w.xn, w.qkv, D.bqkv, qkv_epi);
        } else {
            launch_gemm_f32(D.f_qkv, H, NQ, seq, w.xn, w.qkv, D.bqkv, qkv_epi, st);
        }
        launch_rope_pack(w.qkv, seq, start_pos, nullptr, m->nh, m->nkv, m->hd, m->cos_t, m->sin_t, kv, l, w.q8,
                         w.qsc, st, w.kp, pending_qkv, pending_qkv > 1 ? D.bqkv : nullptr);
        at.layer = l;
        if (split_rows) {
            at.row0 = 0;
            at.nrows = seq;
            launch_attention_prefill_split(at, st);
        } else {
            for (int r0 = 0; r0 < seq; r0 += chunk) {
                at.row0 = r0;
                at.nrows = std::min(chunk, seq - r0);
                launch_attention(at, st);
            }
        }
        if (mixed)
            launch_gemm(D.w[3], seq, w.att, w.X, H, nullptr, EPI_RESID, st);
        else if (q8)
            pending_x = gemm_q8(D.o, D.mo, w.att, w.X, nullptr, EPI_RESID, fuse_x);
        else
            launch_gemm_f32(D.f_o, m->qd, H, seq, w.att, w.X, nullptr, EPI_RESID, st);
        if (!mf) launch_rmsnorm(w.X, w.xn, D.rms2, H, seq, st);
        if (mixed) {
            launch_gemm(D.w[4], seq, w.xn, w.g, F, nullptr, EPI_STORE, st);
            launch_gemm(D.w[6], seq, w.xn, w.u, F, nullptr, EPI_STORE, st);
            launch_silu_mul(w.g, w.u, 0, seq, F, w.h, st);
            launch_gemm(D.w[5], seq, w.h, w.X, H, nullptr, EPI_RESID, st);
        } else if (mf) {
            norm_gemm_q8(D.mgu, D.rms2, w.h, F, nullptr, EPI_SWIGLU);  // h = silu(gate) * up, F wide
            pending_x = gemm_q8(D.down, D.mdown, w.h, w.X, nullptr, EPI_RESID, fuse_x);
        } else if (q8) {
            gemm_q8(D.gu, D.mgu, w.xn, w.g, nullptr, EPI_STORE);
            launch_silu_mul(w.g, nullptr, 1, seq, F, w.h, st);
            gemm_q8(D.down, D.mdown, w.h, w.X, nullptr, EPI_RESID);
        } else {
            launch_gemm_f32(D.f_w1, H, F, seq, w.xn, w.g, nullptr, EPI_STORE, st);
            launch_gemm_f32(D.f_w3, H, F, seq, w.xn, w.u, nullptr, EPI_STORE, st);
            launch_silu_mul(w.g, w.u, 0, seq, F, w.h, st);
            launch_gemm_f32(D.f_w2, F, H, seq, w.h, w.X, nullptr, EPI_RESID, st);
        }
        if (layer_out_host) {
            resolve_x();
            CK(hipMemcpyAsync(layer_out_host + (size_t)l * seq * H, w.X, sizeof(float) * seq * H,
                              hipMemcpyDeviceToHost, st));
            CK(hipStreamSynchronize(st));
        }
    }
    resolve_x();
    CK(hipGetLastError());
}

// attention score scratch (floats) a layer pass over `seq` rows attending up to max_keys keys takes
size_t scores_need(const jyhip_model* m, int seq, int max_keys) {
    return (size_t)m->nh * max_keys * (size_t)std::max(1, std::min(seq, 64));
}

// the layers over workspace w, whose buffers hold `seq` rows and scores_need(seq, max_keys) floats
void run_layers(jyhip_model* m, Workspace& w, const KVDev& kv, int seq, int start_pos, const int* state,
                float* layer_out_host, int max_keys) {
    if (seq == 1)
        run_decode_layers(m, w, kv, state, start_pos, layer_out_host, max_keys);
    else
        run_prefill_layers(m, w, kv, seq, start_pos, layer_out_host, max_keys);
}

// final RMSNorm of the last row + lm_head (+ greedy pick when fused) -> m->logits
// final norm + lm_head (generate.h:48-49): fused into the Q8 matvec's prologue
void final_and_head(jyhip_model* m, Workspace& w, const float* xlast, bool argmax, int neos) {
    if (m->wtype == JY_Q8_0) {
        MvArgs a;
        if (argmax) {
            a.ids = m->ids;
            a.mstate = m->state;
            a.eos = m->eos;
            a.neos = neos;
            a.part_val = m->part_val;
            a.part_idx = m->part_idx;
        }
        q8_matvec(m, m->lm_q8, xlast, m->final_rms, m->logits, argmax ? EPI_ARGMAX : EPI_STORE, a, m->stream);
    } else if (m->wtype == WT_MIXED) {
        launch_rmsnorm(xlast, w.xn, m->final_rms, m->H, 1, m->stream);
        launch_mv(m->lm_w, w.xn, m->logits, EPI_STORE, nullptr, m->stream);
    } else {
        launch_rmsnorm(xlast, w.xn, m->final_rms, m->H, 1, m->stream);
        launch_matvec_f32(m->lm_f32, m->H, m->V, w.xn, m->logits, nullptr, EPI_STORE, m->stream);
    }
}

// greedy pick: fused into lm_head when possible, else the standalone kernel
// (repetition penalty, f32 models)
void head_and_pick(jyhip_model* m, Workspace& w, const float* xlast, bool greedy, float rp, int prompt_len,
                   int neos) {
    const bool fused = greedy && rp == 1.0f && m->wtype == JY_Q8_0;
    final_and_head(m, w, xlast, fused, neos);
    if (greedy && !fused) launch_argmax(m->logits, m->V, m->ids, m->state, m->eos, neos, rp, prompt_len, m->stream);
}

// embedding rows of ids[id0 + i] (or ids[state[0]-1]) into X
void embed_rows(jyhip_model* m, int id0, const int* state, int seq, float* X) {
    if (m->wtype == WT_MIXED)
        launch_embed_w(m->embed_w, m->H, m->ids, id0, state, seq, X, m->stream);
    else
        launch_embed(m->wtype == JY_Q8_0 ? &m->embed_q8 : nullptr, m->embed_f32, m->H, m->ids, id0, state, seq, X,
                     m->stream);
}

// one decode step: embed ids[len-1], layers, final norm, lm_head, greedy pick
// short_ctx: the step will only be replayed at sequence lengths up to short_keys(m)
void decode_step(jyhip_model* m, const KVDev& kv, int max_keys, bool greedy, float rp, int prompt_len, int neos,
                 bool short_ctx) {
    Workspace& w = m->ws;
    embed_rows(m, 0, m->state, 1, w.X);
    if (use_persist(m)) {
        const bool fused = greedy && rp == 1.0f;  // the kernel's own lm_head and greedy pick
        launch_persist(m, w, kv, m->state, 0, max_keys, nullptr, fused, neos);
        if (!fused) head_and_pick(m, w, w.X, greedy, rp, prompt_len, neos);
        return;
    }
    run_decode_layers(m, w, kv, m->state, 0, nullptr, max_keys, short_ctx);
    head_and_pick(m, w, w.X, greedy, rp, prompt_len, neos);
}

// temperature sampling and the repetition penalty on the host, as generate.h:50-77
int host_pick(jyhip_model* m, std::vector<float>& logits, const std::vector<int>& ids, int len, int prompt_len,
              float temperature, float rp, unsigned& rng) {
    const int V = m->V;
    if (rp != 1.0f)
        for (int i = prompt_len; i < len; i++) {
            const int id = ids[i];
            if (id >= 0 && id < V) logits[id] = logits[id] > 0.0f ? logits[id] / rp : logits[id] * rp;
        }
    int next = 0;
    if (temperature <= 0.0f) {
        for (int v = 1; v < V; v++)
            if (logits[v] > logits[next]) next = v;
        return next;
    }
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
    return next;
}
// ---- captured decode graphs: what a replay addresses, checked on the host
//
// A replayed graph keeps the device addresses its kernels were captured with.  At capture
// the graph is walked (kernel nodes only, one chain of dependencies as a single stream
// records it, launch shapes within the device's limits), and every device buffer the decode
// step can address is listed and checked to be a live device allocation on the model's
// device.  Before each run of replays the list is compared with the buffers the model and
// cache hold then, so a buffer replaced since capture (a grown workspace, a new cache) is
// found on the host instead of being read on the device.

// every device buffer a decode step of m over kv may address (a superset: unused ones too)
std::vector<const void*> step_buffers(const jyhip_model* m, const KVDev& kv) {
    std::vector<const void*> b;
    auto add = [&](const void* p) {
        if (p) b.push_back(p);
    };
    auto q8 = [&](const Q8Dev& q) {
        add(q.qs);
        add(q.d);
    };
    auto dw = [&](const DevW& w) {
        add(w.dense);
        q8(w.q8);
        add(w.kq.nib);
        add(w.kq.hi);
        add(w.kq.hdr);
        add(w.kq.dm);
    };
    const Workspace& w = m->ws;
    for (const void* p : {(const void*)w.X, (const void*)w.xn, (const void*)w.qkv, (const void*)w.att,
                          (const void*)w.g, (const void*)w.u, (const void*)w.h, (const void*)w.q8,
                          (const void*)w.qsc, (const void*)w.scores, (const void*)w.part, (const void*)w.ah,
                          (const void*)w.al, (const void*)w.aus})
        add(p);
    for (const void* p : {(const void*)m->cos_t, (const void*)m->sin_t, (const void*)m->embed_f32,
                          (const void*)m->lm_f32, (const void*)m->final_rms, (const void*)m->logits,
                          (const void*)m->ids, (const void*)m->state, (const void*)m->eos, (const void*)m->part_val,
                          (const void*)m->part_idx, (const void*)m->pk_layers, (const void*)m->pk_flags,
                          (const void*)m->pk_err})
        add(p);
    q8(m->embed_q8);
    q8(m->lm_q8);
    dw(m->embed_w);
    dw(m->lm_w);
    for (const DevLayer& D : m->layers) {
        add(D.rms1);
        add(D.rms2);
        add(D.bqkv);
        q8(D.qkv);
        q8(D.o);
        q8(D.gu);
        q8(D.down);
        for (const void* p : {(const void*)D.f_qkv, (const void*)D.f_o, (const void*)D.f_w1, (const void*)D.f_w3,
                              (const void*)D.f_w2})
            add(p);
        for (const DevW& x : D.w) dw(x);
    }
    add(kv.k);
    add(kv.v);
    add(kv.ks);
    add(kv.vs);
    return b;
}

// what the walk of one captured graph found
struct GraphCheck {
    size_t nodes = 0, edges = 0, buffers = 0;
};

// the graph's shape and the buffers' liveness; throws with what is wrong
GraphCheck check_graph(hipGraph_t graph, const jyhip_model* m, const std::vector<const void*>& bufs) {
    GraphCheck r;
    size_t n = 0;
    CK(hipGraphGetNodes(graph, nullptr, &n));
    std::vector<hipGraphNode_t> nodes(n);
    if (n) CK(hipGraphGetNodes(graph, nodes.data(), &n));
    size_t ne = 0;
    CK(hipGraphGetEdges(graph, nullptr, nullptr, &ne));
    size_t nroot = 0;
    CK(hipGraphGetRootNodes(graph, nullptr, &nroot));
    if (n == 0) fail("captured decode graph: no nodes");
    if (ne != n - 1 || nroot != 1)
        fail("captured decode graph: not one chain (" + std::to_string(n) + " nodes, " + std::to_string(ne) +
             " edges, " + std::to_string(nroot) + " roots)");
    for (size_t i = 0; i < n; i++) {
        hipGraphNodeType t;
        CK(hipGraphNodeGetType(nodes[i], &t));
        if (t != hipGraphNodeTypeKernel)
            fail("captured decode graph: node " + std::to_string(i) + " is not a kernel (type " + std::to_string((int)t) +
                 ")");
        hipKernelNodeParams kp{};
        CK(hipGraphKernelNodeGetParams(nodes[i], &kp));
        const size_t grid = (size_t)kp.gridDim.x * kp.gridDim.y * kp.gridDim.z;
        const size_t block = (size_t)kp.blockDim.x * kp.blockDim.y * kp.blockDim.z;
        if (!kp.func || grid == 0 || block == 0 || block > 1024 || kp.sharedMemBytes > 160u * 1024u ||
            (!kp.kernelParams && !kp.extra))
            fail("captured decode graph: kernel node " + std::to_string(i) + " has an invalid launch (grid " +
                 std::to_string(grid) + ", block " + std::to_string(block) + ", LDS " +
                 std::to_string(kp.sharedMemBytes) + ")");
    }
    for (const void* p : bufs) {
        hipPointerAttribute_t a{};
        const hipError_t e = hipPointerGetAttributes(&a, p);
        if (e != hipSuccess || a.type != hipMemoryTypeDevice || a.device != m->device) {
            (void)hipGetLastError();
            char buf[64];
            snprintf(buf, sizeof buf, "%p", p);
            fail(std::string("captured decode graph: buffer ") + buf + " is not a live allocation on device " +
                 std::to_string(m->device));
        }
    }
    r.nodes = n;
    r.edges = ne;
    r.buffers = bufs.size();
    return r;
}

// One generation (generate_cached, libs/model_libs/generate.h:9-89) driven step by
// step: begin() runs the prompt and picks the first token, step(n) produces up to
// n more.  Greedy decoding stays on the device (ids and the sequence length live
// in device memory), so a run of steps is a run of graph launches with no host
// round trip unless eos ids, a callback or sampling need one.
struct Session {
    jyhip_model* m = nullptr;
    jyhip_kv* kv = nullptr;
    bool kv_owned = false;
    int plen = 0, max_seq = 0, total = 0, len = 0, max_keys = 0, neos = 0;
    float temperature = 0.0f, rp = 1.0f;
    bool greedy = true, stopped = false, done_early = false;
    std::vector<int> ids, eos;
    unsigned rng = 12345u;
    jyhip_token_cb cb = nullptr;
    void* ud = nullptr;
    // the decode step as a graph: [1] for sequence lengths up to short_keys(m) (one
    // attention kernel), [0] past it; each captured the first time a step call needs it
    hipGraphExec_t exec[2] = {nullptr, nullptr};
    unsigned exec_gen[2] = {0, 0};  // the workspace generation each graph was captured on
    int exec_mode[2] = {0, 0};      // the model's mode each graph was captured in
    std::vector<const void*> exec_bufs[2];  // the buffers each graph may address, at capture
    GraphCheck exec_check[2];
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    double decode_ms = 0.0;
    int decoded = 0;
    std::vector<float> hlog;
    float* logits_out = nullptr;

    ~Session() {
        for (hipGraphExec_t e : exec)
            if (e) (void)hipGraphExecDestroy(e);
        if (m && m->owner == this) m->owner = nullptr;
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
        if (kv_owned && kv) jyhip_kv_free(kv);
    }

    bool is_eos(int id) const {
        for (int e : eos)
            if (id == e) return true;
        return false;
    }

    // sampling / penalty on the host (generate.h:50-77); writes the pick back
    int pick_host() {
        hipStream_t st = m->stream;
        hlog.resize(m->V);
        CK(hipMemcpyAsync(hlog.data(), m->logits, sizeof(float) * m->V, hipMemcpyDeviceToHost, st));
        CK(hipStreamSynchronize(st));
        if (logits_out) memcpy(logits_out, hlog.data(), sizeof(float) * m->V);
        const int next = host_pick(m, hlog, ids, len, plen, temperature, rp, rng);
        const int s2[2] = {len + 1, 0};
        CK(hipMemcpyAsync(m->ids + len, &next, sizeof(int), hipMemcpyHostToDevice, st));
        CK(hipMemcpyAsync(m->state, s2, sizeof(s2), hipMemcpyHostToDevice, st));
        CK(hipStreamSynchronize(st));
        return next;
    }

    int fetch_last() {
        int v[2];
        CK(hipMemcpyAsync(v, m->state, sizeof(v), hipMemcpyDeviceToHost, m->stream));
        CK(hipStreamSynchronize(m->stream));
        int id = 0;
        CK(hipMemcpy(&id, m->ids + v[0] - 1, sizeof(int), hipMemcpyDeviceToHost));
        return id;
    }

    void accept(int next) {
        ids[len++] = next;
        if (cb && cb(next, ud)) stopped = true;
        if (is_eos(next)) stopped = true;
    }

    // returns false when generate() would return before the loop (generate.h:25-32)
    bool begin(jyhip_model* model, jyhip_kv* kv_in, const int* prompt, int plen_, const int* eos_ids, int neos_,
               int max_seq_, int max_new, float temperature_, float rp_, jyhip_token_cb cb_, void* ud_,
               int* prompt_out, bool resume = false) {
        m = model;
        plen = plen_;
        max_seq = max_seq_;
        temperature = temperature_;
        rp = rp_;
        cb = cb_;
        ud = ud_;
        if (!prompt) fail("prompt_ids is NULL");
        if (plen <= 0 || plen > max_seq) return false;  // generate.h:25
        if (max_seq > m->max_seq) fail("max_seq exceeds the model's RoPE table (jyhip_model_upload max_seq)");
        if (neos_ < 0 || (neos_ > 0 && !eos_ids)) fail("bad eos list");
        if (neos_ > m->eos_cap) fail("too many eos ids");
        for (int i = 0; i < plen; i++)
            if (prompt[i] < 0 || prompt[i] >= m->V) fail("prompt id out of vocabulary");
        if (resume && !kv_in) fail("resume: no KV cache given");
        if (kv_in) {
            kv = kv_in;
            if (kv->dev.num_layers < m->L || kv->dev.max_seq < max_seq || kv->dev.nkv != m->nkv || kv->dev.hd != m->hd)
                fail("generate: KV cache shape does not match the model");
            if (kv->device != m->device) fail("generate: the KV cache is on another device than the model");
        } else {
            kv = jyhip_kv_create(m, max_seq);
            if (!kv) fail(g_err);
            kv_owned = true;
        }
        neos = neos_;
        eos.assign(eos_ids, eos_ids + neos);
        ids.assign(prompt, prompt + plen);
        ids.resize((size_t)max_seq + 1);
        if (prompt_out)
            for (int i = 0; i < plen; i++) prompt_out[i] = prompt[i];
        len = plen;
        // positions [0, keep) of the prompt are already in the cache (resume); the rest run
        // as one chunk at start_pos = keep, as forward_cached does (forward.h:95)
        const int keep = resume ? kv->current_len : 0;
        if (keep < 0 || keep >= plen) fail("resume: the cache must hold fewer positions than the prompt");
        kv->current_len = keep;
        if (max_new <= 0) return false;                  // generate.h:32
        total = std::min(max_new, max_seq - plen);        // tokens this generation may produce
        if (total <= 0) return false;                     // generate.h:39: len < max_seq fails at once
        greedy = temperature <= 0.0f;
        max_keys = (max_seq + 3) / 4 * 4;
        for (hipEvent_t& e : ev) CK(hipEventCreate(&e));

        hipStream_t st = m->stream;
        const int seq = plen - keep;
        ensure_ws(m, seq);
        ensure_scores(m, scores_need(m, seq, max_keys));
        ensure_part(m, part_need(m, max_keys));
        if (seq > 1 && use_mfma(m)) {  // (allocated here, before the prompt step is timed)
            ensure_split(m, mfma_split_halves(m, seq), mfma_rows_padded(seq));
            ensure_kpart(m, mfma_kpart_need(m, seq));
        }
        m->owner = this;
        CK(hipMemcpyAsync(m->ids, prompt, sizeof(int) * plen, hipMemcpyHostToDevice, st));
        const int st0[4] = {plen, 0, 0, 0};
        CK(hipMemcpyAsync(m->state, st0, sizeof(st0), hipMemcpyHostToDevice, st));
        if (neos) CK(hipMemcpyAsync(m->eos, eos_ids, sizeof(int) * neos, hipMemcpyHostToDevice, st));
        // step 0: the prompt (generate.h:43-49 with seq = prompt_len)
        CK(hipEventRecord(ev[0], st));
        Workspace& w = m->ws;
        embed_rows(m, keep, nullptr, seq, w.X);
        run_layers(m, w, kv->dev, seq, keep, nullptr, nullptr, max_keys);
        head_and_pick(m, w, w.X + (size_t)(seq - 1) * m->H, greedy, rp, plen, neos);
        CK(hipEventRecord(ev[1], st));
        CK(hipGetLastError());
        accept(greedy ? fetch_last() : pick_host());
        return true;
    }

    int remaining() const { return stopped ? 0 : plen + total - len; }

    void capture(int which) {
        hipStream_t st = m->stream;
        hipGraph_t graph = nullptr;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        try {
            decode_step(m, kv->dev, max_keys, greedy, rp, plen, neos, which == 1);
        } catch (...) {
            (void)hipStreamEndCapture(st, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            throw;
        }
        CK(hipStreamEndCapture(st, &graph));
        std::vector<const void*> bufs = step_buffers(m, kv->dev);
        GraphCheck gc;
        try {
            gc = check_graph(graph, m, bufs);
        } catch (...) {
            (void)hipGraphDestroy(graph);
            throw;
        }
        const hipError_t ie = hipGraphInstantiate(&exec[which], graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        ck(ie, "hipGraphInstantiate");
        exec_gen[which] = m->ws.gen;
        exec_mode[which] = m->mode;
        exec_bufs[which] = std::move(bufs);
        exec_check[which] = gc;
    }

    // the buffers graph `which` was captured with are the ones the model and cache hold now
    void check_buffers(int which) const {
        if (!exec[which]) return;
        if (step_buffers(m, kv->dev) != exec_bufs[which])
            fail("session: a buffer the captured decode graph addresses was replaced after capture");
    }

    // the graph for a step over a sequence of `length` tokens (it attends `length` keys)
    hipGraphExec_t graph_for(int length) const { return exec[length <= short_keys(m) ? 1 : 0]; }

    // up to n more tokens; returns how many were produced
    int step(int n) {
        n = std::min(n, remaining());
        if (n <= 0) return 0;
        if (m->owner != this)
            fail("session: a later generation has started on this model; this one can no longer step");
        // a graph captured before the workspace was replaced (a longer prompt or chunk
        // since) would address freed buffers: capture it again
        ensure_part(m, part_need(m, max_keys));  // the mode may have changed since begin
        for (int i = 0; i < 2; i++)
            if (exec[i] && (exec_gen[i] != m->ws.gen || exec_mode[i] != m->mode)) {
                (void)hipGraphExecDestroy(exec[i]);
                exec[i] = nullptr;
            }
        // the steps run at lengths len .. len+n-1: capture what they need up front
        if (len <= short_keys(m) && !exec[1]) capture(1);
        if (len + n - 1 > short_keys(m) && !exec[0]) capture(0);
        check_buffers(0);
        check_buffers(1);
        hipStream_t st = m->stream;
        CK(hipEventRecord(ev[2], st));
        int made = 0;
        if (!greedy || cb || neos > 0) {
            for (; made < n && !stopped; made++) {
                CK(hipGraphLaunch(graph_for(len), st));
                accept(greedy ? fetch_last() : pick_host());
            }
        } else {
            for (int s = 0; s < n; s++) CK(hipGraphLaunch(graph_for(len + s), st));
            CK(hipMemcpyAsync(ids.data() + len, m->ids + len, sizeof(int) * n, hipMemcpyDeviceToHost, st));
            made = n;
            len += n;
        }
        CK(hipEventRecord(ev[3], st));
        CK(hipStreamSynchronize(st));
        check_persist(m);
        float ms = 0.0f;
        CK(hipEventElapsedTime(&ms, ev[2], ev[3]));
        decode_ms += ms;
        decoded += made;
        return made;
    }

    double prefill_ms() {
        float ms = 0.0f;
        CK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        return ms;
    }

    void finish() { kv->current_len = len - 1; }  // K/V of the last token is never computed
};

int generate_impl(jyhip_model* m, jyhip_kv* kv_in, const int* prompt, int plen, const int* eos, int neos,
                  int max_seq, int max_new, float temperature, float rp, int* out_ids, jyhip_token_cb cb, void* ud,
                  float* logits_out, jyhip_stats* stats) {
    if (stats) *stats = jyhip_stats{};
    if (!out_ids) fail("out_ids is NULL");
    Session s;
    s.logits_out = logits_out;
    if (!s.begin(m, kv_in, prompt, plen, eos, neos, max_seq, max_new, temperature, rp, cb, ud, out_ids))
        return (plen <= 0 || plen > max_seq) ? 0 : plen;
    while (s.remaining() > 0) s.step(s.remaining());
    s.finish();
    if (logits_out && s.greedy)
        CK(hipMemcpy(logits_out, m->logits, sizeof(float) * m->V, hipMemcpyDeviceToHost));
    for (int i = plen; i < s.len; i++) out_ids[i] = s.ids[i];
    if (stats) {
        stats->prefill_ms = s.prefill_ms();
        stats->decode_ms = s.decode_ms;
        stats->prompt_len = plen;
        stats->decoded = s.decoded;
        stats->upload_ms = m->upload_ms;
    }
    return s.len;
}


int forward_impl(jyhip_model* m, jyhip_kv* kv, float* X, int seq, int start_pos, float* layer_out) {
    if (!kv || !X) fail("forward: NULL kv or X");
    if (kv->dev.num_layers < m->L || kv->dev.nkv != m->nkv || kv->dev.hd != m->hd)
        fail("forward: KV cache shape does not match the model");  // forward.h:60-61
    if (kv->device != m->device) fail("forward: the KV cache is on another device than the model");
    if (start_pos < 0) fail("forward: start_pos must not be negative");
    if (seq <= 0) fail("forward: seq must be positive");
    if ((size_t)start_pos + seq > (size_t)kv->dev.max_seq) fail("forward: KV cache capacity exceeded");
    if (start_pos + seq > m->max_seq) fail("forward: position beyond the RoPE table");
    hipStream_t st = m->stream;
    const int max_keys = (start_pos + seq + 3) / 4 * 4;
    ensure_ws(m, seq);
    ensure_scores(m, scores_need(m, seq, max_keys));
    ensure_part(m, part_need(m, max_keys));
    Workspace& w = m->ws;
    CK(hipMemcpyAsync(w.X, X, sizeof(float) * seq * m->H, hipMemcpyHostToDevice, st));
    run_layers(m, w, kv->dev, seq, start_pos, nullptr, layer_out, max_keys);
    launch_rmsnorm(w.X, w.xn, m->final_rms, m->H, seq, st);  // forward.h:86-94
    CK(hipGetLastError());
    CK(hipMemcpyAsync(X, w.xn, sizeof(float) * seq * m->H, hipMemcpyDeviceToHost, st));
    CK(hipStreamSynchronize(st));
    check_persist(m);
    kv->current_len = start_pos + seq;
    return 0;
}

// The workspace buffers for `seq` rows and `scores_n` score floats laid out in
// [base, base + *bytes), each buffer 256-byte aligned (the same buffers ensure_ws and
// ensure_scores allocate one by one).
Workspace ws_view(const jyhip_model* m, int seq, int max_keys, size_t scores_n, unsigned char* base,
                  size_t* bytes) {
    size_t off = 0;
    auto take = [&](size_t nbytes) {
        unsigned char* p = base + off;
        off += (std::max<size_t>(nbytes, 1) + 255) / 256 * 256;
        return p;
    };
    const size_t r = (size_t)seq;
    Workspace w;
    w.X = (float*)take(r * m->H * 4);
    w.xn = (float*)take(r * m->H * 4);
    w.qkv = (float*)take(r * (m->qd + 2 * m->kvd) * 4);
    w.att = (float*)take(r * m->qd * 4);
    w.g = (float*)take(r * 2 * m->F * 4);
    w.u = (float*)take(r * m->F * 4);
    w.h = (float*)take(r * m->F * 4);
    w.q8 = (int8_t*)take(r * m->qd);
    w.qsc = (float*)take(r * m->nh * 4);
    w.scores = (float*)take(scores_n * 4);
    w.scores_n = scores_n;
    w.part_n = part_need(m, max_keys);
    w.part = (float*)take(w.part_n * 4);
    if (seq > 1 && use_mfma(m)) {
        w.a_cap = mfma_split_halves(m, seq);
        w.a_rows = mfma_rows_padded(seq);
        w.ah = (_Float16*)take(w.a_cap * 2);
        w.al = (_Float16*)take(w.a_cap * 2);
        w.aus = (float*)take((size_t)w.a_rows * 4);
        w.kp_n = mfma_kpart_need(m, seq);
        w.kp = (float*)take(w.kp_n * 4);
    }
    w.rows = seq;
    *bytes = off;
    return w;
}

// forward_cached over the GPU's static scratch: the checks and steps of forward_impl
// (layer outputs aside) with no device allocation
int forward_noalloc(jyhip_model* m, jyhip_kv* kv, float* X, int seq, int start_pos) {
    if (!kv || !X) fail("forward: NULL kv or X");
    if (kv->dev.num_layers < m->L || kv->dev.nkv != m->nkv || kv->dev.hd != m->hd)
        fail("forward: KV cache shape does not match the model");
    if (kv->device != m->device) fail("forward: the KV cache is on another device than the model");
    if (start_pos < 0) fail("forward: start_pos must not be negative");
    if (seq <= 0) fail("forward: seq must be positive");
    if ((size_t)start_pos + seq > (size_t)kv->dev.max_seq) fail("forward: KV cache capacity exceeded");
    if (start_pos + seq > m->max_seq) fail("forward: position beyond the RoPE table");
    unsigned char* base = static_cast<unsigned char*>(g_scratch[m->device]);
    if (!base) fail("forward_cached_noalloc: the device's scratch address is not set up");
    const int max_keys = (start_pos + seq + 3) / 4 * 4;
    size_t need = 0;
    Workspace w = ws_view(m, seq, max_keys, scores_need(m, seq, max_keys), base, &need);
    if (need > (size_t)JYHIP_NOALLOC_SCRATCH_BYTES)
        fail("forward_cached_noalloc: " + std::to_string(seq) + " rows attending " + std::to_string(start_pos + seq) +
             " keys need " + std::to_string(need) + " bytes of workspace, more than the " +
             std::to_string((size_t)JYHIP_NOALLOC_SCRATCH_BYTES) + "-byte static scratch");
    hipStream_t st = m->stream;
    // the allocating path starts from zeroed buffers; so does this one, whatever an
    // earlier call left in the shared array
    launch_zero_fill(base, need, st);
    CK(hipMemcpyAsync(w.X, X, sizeof(float) * seq * m->H, hipMemcpyHostToDevice, st));
    run_layers(m, w, kv->dev, seq, start_pos, nullptr, nullptr, max_keys);
    launch_rmsnorm(w.X, w.xn, m->final_rms, m->H, seq, st);  // forward.h:86-94
    CK(hipGetLastError());
    CK(hipMemcpyAsync(X, w.xn, sizeof(float) * seq * m->H, hipMemcpyDeviceToHost, st));
    CK(hipStreamSynchronize(st));
    check_persist(m);
    kv->current_len = start_pos + seq;
    return 0;
}

template <class F>
auto guarded(F&& f, decltype(f()) bad) -> decltype(f()) {
    try {
        g_err.clear();
        return f();
    } catch (const Error& e) {
        g_err = e.msg;
    } catch (const std::exception& e) {
        g_err = e.what();
    } catch (...) {
        g_err = "unknown error";
    }
    return bad;
}

}  // namespace

extern "C" {

JYHIP_API const char* jyhip_last_error(void) { return g_err.c_str(); }

JYHIP_API int jyhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

JYHIP_API int jyhip_set_device(int device) {
    return guarded([&]() {
        CK(hipSetDevice(device));
        return 0;
    }, -1);
}

JYHIP_API jyhip_model* jyhip_model_upload(const jy_model_desc* d, int max_seq) {
    return guarded([&]() -> jyhip_model* {
        const int wtype = check_desc(d);
        if (max_seq <= 0) fail("max_seq must be positive");
        jyhip_model* m = new jyhip_model();
        try {
            CK(hipGetDevice(&m->device));
            init_device_kernels(m->device);
            const auto t0 = std::chrono::steady_clock::now();
            upload(m, d, max_seq, wtype);
            CK(hipDeviceSynchronize());
            m->upload_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        } catch (...) {
            release(m);
            throw;
        }
        return m;
    }, nullptr);
}

JYHIP_API void jyhip_model_free(jyhip_model* m) { release(m); }

JYHIP_API size_t jyhip_model_weight_bytes(const jyhip_model* m) { return m ? m->weight_bytes : 0; }

JYHIP_API int jyhip_model_set_mode(jyhip_model* m, int mode) {
    return guarded([&]() {
        if (!m) fail("model is NULL");
        if (mode & ~JYHIP_MODE_ALL) fail("unknown mode bits");
        if (mode & JYHIP_MODE_MFMA_PREFILL) {
            CK(hipSetDevice(m->device));
            build_mfma(m);
        }
        m->mode = mode;
        return 0;
    }, -1);
}

JYHIP_API int jyhip_model_mode(const jyhip_model* m) { return m ? m->mode : -1; }

JYHIP_API double jyhip_model_upload_ms(const jyhip_model* m) { return m ? m->upload_ms : 0.0; }

JYHIP_API jyhip_kv* jyhip_kv_create(const jyhip_model* m, int max_seq) {
    return guarded([&]() -> jyhip_kv* {
        if (!m) fail("model is NULL");
        if (max_seq <= 0) fail("max_seq must be positive");
        jyhip_kv* kv = new jyhip_kv();
        KVDev& k = kv->dev;
        k.num_layers = m->L;
        k.max_seq = max_seq;
        k.nkv = m->nkv;
        k.hd = m->hd;
        const size_t n = (size_t)m->L * m->nkv * max_seq * m->hd, rows = (size_t)m->L * m->nkv * max_seq;
        try {
            k.k = dalloc<int8_t>(n);
            k.v = dalloc<int8_t>(n);
            k.ks = dalloc<float>(rows);
            k.vs = dalloc<float>(rows);
        } catch (...) {
            dfree(k.k);
            dfree(k.v);
            dfree(k.ks);
            dfree(k.vs);
            delete kv;
            throw;
        }
        kv->device = m->device;
        return kv;
    }, nullptr);
}

JYHIP_API void jyhip_kv_free(jyhip_kv* kv) {
    if (!kv) return;
    (void)hipDeviceSynchronize();
    dfree(kv->dev.k);
    dfree(kv->dev.v);
    dfree(kv->dev.ks);
    dfree(kv->dev.vs);
    delete kv;
}

JYHIP_API int jyhip_kv_len(const jyhip_kv* kv) { return kv ? kv->current_len : -1; }

JYHIP_API int jyhip_kv_set_len(jyhip_kv* kv, int n) {
    return guarded([&]() {
        if (!kv) fail("kv is NULL");
        if (n < 0 || n > kv->dev.max_seq) fail("length outside the cache");
        kv->current_len = n;
        return 0;
    }, -1);
}

static void kv_range(const jyhip_kv* kv, int layer, int pos0, int npos) {
    if (!kv) fail("kv is NULL");
    if (layer < 0 || layer >= kv->dev.num_layers) fail("layer out of range");
    if (pos0 < 0 || npos < 0 || (size_t)pos0 + npos > (size_t)kv->dev.max_seq) fail("positions out of range");
}

JYHIP_API int jyhip_kv_write(jyhip_kv* kv, int layer, int pos0, int npos, const int8_t* k, const float* ks,
                             const int8_t* v, const float* vs) {
    return guarded([&]() {
        kv_range(kv, layer, pos0, npos);
        if (npos == 0) return 0;
        if (!k || !ks || !v || !vs) fail("NULL buffer");
        const size_t n = (size_t)npos * kv->dev.nkv * kv->dev.hd, r = (size_t)npos * kv->dev.nkv;
        int8_t *dk = dalloc<int8_t>(n, false), *dv = dalloc<int8_t>(n, false);
        float *dks = dalloc<float>(r, false), *dvs = dalloc<float>(r, false);
        hipError_t e = hipMemcpy(dk, k, n, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(dv, v, n, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(dks, ks, r * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(dvs, vs, r * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) {
            launch_kv_import(dk, dks, dv, dvs, pos0, npos, kv->dev, layer, nullptr);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipDeviceSynchronize();
        dfree(dk);
        dfree(dv);
        dfree(dks);
        dfree(dvs);
        ck(e, "kv_write");
        return 0;
    }, -1);
}

JYHIP_API int jyhip_kv_read(const jyhip_kv* kv, int layer, int pos0, int npos, int8_t* k, float* ks, int8_t* v,
                            float* vs) {
    return guarded([&]() {
        kv_range(kv, layer, pos0, npos);
        if (npos == 0) return 0;
        if (!k || !ks || !v || !vs) fail("NULL buffer");
        const size_t n = (size_t)npos * kv->dev.nkv * kv->dev.hd, r = (size_t)npos * kv->dev.nkv;
        int8_t *dk = dalloc<int8_t>(n, false), *dv = dalloc<int8_t>(n, false);
        float *dks = dalloc<float>(r, false), *dvs = dalloc<float>(r, false);
        launch_kv_export(dk, dks, dv, dvs, pos0, npos, kv->dev, layer, nullptr);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e == hipSuccess) e = hipMemcpy(k, dk, n, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(v, dv, n, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(ks, dks, r * 4, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(vs, dvs, r * 4, hipMemcpyDeviceToHost);
        dfree(dk);
        dfree(dv);
        dfree(dks);
        dfree(dvs);
        ck(e, "kv_read");
        return 0;
    }, -1);
}

JYHIP_API int jyhip_forward_cached(jyhip_model* m, jyhip_kv* kv, float* X, int seq, int start_pos, float* layer_out) {
    return guarded([&]() {
        if (!m) fail("model is NULL");
        return forward_impl(m, kv, X, seq, start_pos, layer_out);
    }, -1);
}

JYHIP_API int jyhip_forward_cached_noalloc(jyhip_model* m, jyhip_kv* kv, float* X, int seq, int start_pos) {
    return guarded([&]() {
        if (!m) fail("model is NULL");
        return forward_noalloc(m, kv, X, seq, start_pos);
    }, -1);
}

JYHIP_API int jyhip_generate(jyhip_model* m, jyhip_kv* kv, const int* prompt_ids, int prompt_len, const int* eos_ids,
                             int num_eos, int max_seq, int max_new, float temperature, float repetition_penalty,
                             int* out_ids, jyhip_token_cb cb, void* cb_ud, float* logits_out, jyhip_stats* stats) {
    return guarded([&]() {
        if (!m) fail("model is NULL");
        return generate_impl(m, kv, prompt_ids, prompt_len, eos_ids, num_eos, max_seq, max_new, temperature,
                             repetition_penalty, out_ids, cb, cb_ud, logits_out, stats);
    }, -1);
}

struct jyhip_session {
    Session s;
    bool active = false;  // false: generate() would have returned before its loop
    int result = 0;       // what generate() returns in that case
};

static jyhip_session* session_open(jyhip_model* m, jyhip_kv* kv, const int* prompt_ids, int prompt_len,
                                   const int* eos_ids, int num_eos, int max_seq, int max_new, float temperature,
                                   float repetition_penalty, bool resume) {
    return guarded([&]() -> jyhip_session* {
        if (!m) fail("model is NULL");
        jyhip_session* h = new jyhip_session();
        try {
            h->active = h->s.begin(m, kv, prompt_ids, prompt_len, eos_ids, num_eos, max_seq, max_new, temperature,
                                   repetition_penalty, nullptr, nullptr, nullptr, resume);
            h->result = h->active ? h->s.len : ((prompt_len <= 0 || prompt_len > max_seq) ? 0 : prompt_len);
        } catch (...) {
            delete h;
            throw;
        }
        return h;
    }, nullptr);
}

JYHIP_API jyhip_session* jyhip_session_begin(jyhip_model* m, jyhip_kv* kv, const int* prompt_ids, int prompt_len,
                                             const int* eos_ids, int num_eos, int max_seq, int max_new,
                                             float temperature, float repetition_penalty) {
    return session_open(m, kv, prompt_ids, prompt_len, eos_ids, num_eos, max_seq, max_new, temperature,
                        repetition_penalty, false);
}

JYHIP_API jyhip_session* jyhip_session_resume(jyhip_model* m, jyhip_kv* kv, const int* ids, int n_ids,
                                              const int* eos_ids, int num_eos, int max_seq, int max_new,
                                              float temperature, float repetition_penalty) {
    return session_open(m, kv, ids, n_ids, eos_ids, num_eos, max_seq, max_new, temperature, repetition_penalty,
                        true);
}

JYHIP_API int jyhip_session_step(jyhip_session* h, int n) {
    return guarded([&]() {
        if (!h) fail("session is NULL");
        if (!h->active || n <= 0) return 0;
        const int made = h->s.step(n);
        h->s.finish();
        return made;
    }, -1);
}

JYHIP_API int jyhip_session_remaining(const jyhip_session* h) { return h && h->active ? h->s.remaining() : 0; }

JYHIP_API int jyhip_session_len(const jyhip_session* h) { return !h ? -1 : h->active ? h->s.len : h->result; }

JYHIP_API int jyhip_session_ids(const jyhip_session* h, int* out, int cap) {
    return guarded([&]() {
        if (!h || !out) fail("NULL argument");
        const int n = h->active ? h->s.len : std::min(h->result, (int)h->s.ids.size());
        if (cap < n) fail("output buffer too small");
        for (int i = 0; i < n; i++) out[i] = h->s.ids[i];
        return n;
    }, -1);
}

JYHIP_API int jyhip_session_graph_info(const jyhip_session* h, int which, long long* info) {
    return guarded([&]() {
        if (!h || which < 0 || which > 1 || !info) fail("session_graph_info: bad arguments");
        const Session& s = h->s;
        if (!s.exec[which]) return 0;
        s.check_buffers(which);
        info[0] = (long long)s.exec_check[which].nodes;
        info[1] = (long long)s.exec_check[which].edges;
        info[2] = (long long)s.exec_check[which].buffers;
        return 1;
    }, -1);
}

JYHIP_API int jyhip_session_stats(jyhip_session* h, jyhip_stats* st) {
    return guarded([&]() {
        if (!h || !st) fail("NULL argument");
        *st = jyhip_stats{};
        if (!h->active) return 0;
        st->prefill_ms = h->s.prefill_ms();
        st->decode_ms = h->s.decode_ms;
        st->prompt_len = h->s.plen;
        st->decoded = h->s.decoded;
        st->upload_ms = h->s.m->upload_ms;
        return 0;
    }, -1);
}

JYHIP_API void jyhip_session_end(jyhip_session* h) { delete h; }

JYHIP_API jyhip_q8mat* jyhip_q8_upload(const void* w, int rows, int cols, int copies) {
    return guarded([&]() -> jyhip_q8mat* {
        if (!w || rows <= 0 || cols <= 0 || cols % 32) fail("bad Q8_0 matrix");
        if (copies <= 0) copies = 1;
        jyhip_q8mat* q = new jyhip_q8mat();
        jyhip_model holder;  // borrow q8_alloc's bookkeeping
        try {
            int dev = 0;
            CK(hipGetDevice(&dev));
            init_device_kernels(dev);
            CK(hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking));
            holder.stream = q->stream;
            uint8_t* staging = dalloc<uint8_t>(q8_bytes(rows, cols), false);
            for (int c = 0; c < copies; c++) {
                Q8Dev d = q8_alloc(&holder, rows, cols);
                q8_put(&holder, staging, w, rows, cols, d, 0, 1);
                q->copies.push_back(d);
            }
            dfree(staging);
            q->x = dalloc<float>(cols);
            q->y = dalloc<float>(rows);
        } catch (...) {
            for (void* p : holder.owned) dfree(p);
            if (q->stream) (void)hipStreamDestroy(q->stream);
            delete q;
            throw;
        }
        holder.owned.clear();
        holder.stream = nullptr;
        return q;
    }, nullptr);
}

JYHIP_API void jyhip_q8_free(jyhip_q8mat* q) {
    if (!q) return;
    (void)hipStreamSynchronize(q->stream);
    for (Q8Dev& d : q->copies) {
        dfree(d.qs);
        dfree(d.d);
    }
    for (void* p : q->mowned) dfree(p);
    dfree(q->x);
    dfree(q->y);
    dfree(q->nw);
    (void)hipStreamDestroy(q->stream);
    delete q;
}

JYHIP_API int jyhip_q8_matvec(jyhip_q8mat* q, const float* x, float* y) {
    return guarded([&]() {
        if (!q || !x || !y) fail("NULL argument");
        const Q8Dev& d = q->copies[0];
        CK(hipMemcpyAsync(q->x, x, sizeof(float) * d.cols, hipMemcpyHostToDevice, q->stream));
        if (q->mode & JYHIP_MODE_SPLIT_MV)
            launch_matvec_q8_split(d, q->x, nullptr, q->y, EPI_STORE, MvArgs(), q->stream);
        else
            launch_matvec_q8(d, q->x, nullptr, q->y, EPI_STORE, MvArgs(), q->stream);
        CK(hipGetLastError());
        CK(hipMemcpyAsync(y, q->y, sizeof(float) * d.rows, hipMemcpyDeviceToHost, q->stream));
        CK(hipStreamSynchronize(q->stream));
        return 0;
    }, -1);
}

JYHIP_API int jyhip_q8_set_mode(jyhip_q8mat* q, int mode) {
    return guarded([&]() {
        if (!q) fail("matrix is NULL");
        if (mode & ~(JYHIP_MODE_ALL & ~JYHIP_MODE_PERSIST)) fail("unknown mode bits");
        if ((mode & JYHIP_MODE_MFMA_PREFILL) && q->mcopies.empty()) {
            for (const Q8Dev& d : q->copies) q->mcopies.push_back(mfma_copy(q->mowned, d, q->stream));
            CK(hipStreamSynchronize(q->stream));
        }
        q->mode = mode;
        return 0;
    }, -1);
}

}  // extern "C"

namespace {
// C[mr][rows] = A[mr][cols] W^T for copy c in the matrix's mode, device buffers given;
// the MFMA form splits A into hi / lo first
void q8_gemm_launch(jyhip_q8mat* q, size_t c, int mr, const float* A, float* Cd, _Float16* hi, _Float16* lo,
                    float* us, float* kp, size_t kp_n) {
    const Q8Dev& d = q->copies[c];
    if (q->mode & JYHIP_MODE_MFMA_PREFILL) {
        launch_mfma_split(A, mr, mfma_rows_padded(mr), d.cols, hi, lo, us, q->stream);
        launch_gemm_q8_mfma(q->mcopies[c], mr, hi, lo, us, Cd, d.rows, nullptr, EPI_STORE, q->stream, kp, kp_n);
    } else {
        launch_gemm_q8(d, mr, A, Cd, nullptr, EPI_STORE, q->stream);
    }
}

// the device buffers of a GEMM over mr rows: A, C, the activation split and the partial sums
struct GemmBufs {
    float *A = nullptr, *C = nullptr;
    _Float16 *hi = nullptr, *lo = nullptr;
    float* us = nullptr;
    float* kp = nullptr;
    size_t kp_n = 0;
};

// run f(bufs) with device buffers for mr rows of A uploaded from host
template <class F>
void with_gemm_buffers(jyhip_q8mat* q, int mr, const float* A, F&& f) {
    const Q8Dev& d = q->copies[0];
    const size_t mp = (size_t)mfma_rows_padded(mr);
    GemmBufs b;
    auto free_all = [&]() {
        for (void* p : {(void*)b.A, (void*)b.C, (void*)b.hi, (void*)b.lo, (void*)b.us, (void*)b.kp}) dfree(p);
    };
    try {
        b.A = dalloc<float>((size_t)mr * d.cols, false);
        b.C = dalloc<float>((size_t)mr * d.rows, false);
        b.hi = reinterpret_cast<_Float16*>(dalloc<uint16_t>(mp * d.cols, false));
        b.lo = reinterpret_cast<_Float16*>(dalloc<uint16_t>(mp * d.cols, false));
        b.us = dalloc<float>(mp, false);
        if (!q->mcopies.empty()) b.kp_n = gemm_q8_mfma_kpart_floats(q->mcopies[0], mr, EPI_STORE);
        if (b.kp_n) b.kp = dalloc<float>(b.kp_n, false);
        CK(hipMemcpyAsync(b.A, A, sizeof(float) * mr * d.cols, hipMemcpyHostToDevice, q->stream));
        f(b);
    } catch (...) {
        (void)hipStreamSynchronize(q->stream);
        free_all();
        throw;
    }
    (void)hipStreamSynchronize(q->stream);
    free_all();
}
}  // namespace

extern "C" {

JYHIP_API int jyhip_q8_gemm(jyhip_q8mat* q, int mr, const float* A, float* Cout) {
    return guarded([&]() {
        if (!q || !A || !Cout || mr <= 0) fail("bad argument");
        with_gemm_buffers(q, mr, A, [&](const GemmBufs& b) {
            q8_gemm_launch(q, 0, mr, b.A, b.C, b.hi, b.lo, b.us, b.kp, b.kp_n);
            CK(hipGetLastError());
            CK(hipMemcpyAsync(Cout, b.C, sizeof(float) * mr * q->copies[0].rows, hipMemcpyDeviceToHost, q->stream));
            CK(hipStreamSynchronize(q->stream));
        });
        return 0;
    }, -1);
}

JYHIP_API int jyhip_q8_gemm_time(jyhip_q8mat* q, int mr, const float* A, int iters, double* avg_us) {
    return guarded([&]() {
        if (!q || !A || !avg_us || mr <= 0 || iters <= 0) fail("bad argument");
        with_gemm_buffers(q, mr, A, [&](const GemmBufs& g) {
            for (size_t c = 0; c < q->copies.size(); c++) q8_gemm_launch(q, c, mr, g.A, g.C, g.hi, g.lo, g.us, g.kp, g.kp_n);
            hipEvent_t a, b;
            CK(hipEventCreate(&a));
            CK(hipEventCreate(&b));
            CK(hipEventRecord(a, q->stream));
            for (int i = 0; i < iters; i++)
                q8_gemm_launch(q, (size_t)i % q->copies.size(), mr, g.A, g.C, g.hi, g.lo, g.us, g.kp, g.kp_n);
            CK(hipEventRecord(b, q->stream));
            CK(hipEventSynchronize(b));
            float ms = 0.0f;
            CK(hipEventElapsedTime(&ms, a, b));
            (void)hipEventDestroy(a);
            (void)hipEventDestroy(b);
            CK(hipGetLastError());
            *avg_us = 1000.0 * ms / iters;
        });
        return 0;
    }, -1);
}

JYHIP_API int jyhip_q8_matvec_time(jyhip_q8mat* q, const float* x, int variant, int iters, double* avg_us) {
    return guarded([&]() {
        if (!q || !x || !avg_us || iters <= 0 || variant < 0 || variant > 4) fail("bad argument");
        const Q8Dev& d0 = q->copies[0];
        if ((variant & 1 || variant == 4) && d0.rows % 2) fail("the gate/up variant needs interleaved row pairs");
        const bool split = variant == 2 || variant == 3, lin = variant == 4;
        auto mv = [&](const Q8Dev& W, const float* nw, Epi epi) {
            if (split)
                launch_matvec_q8_split(W, q->x, nw, q->y, epi, MvArgs(), q->stream);
            else
                launch_matvec_q8(W, q->x, nw, q->y, epi, MvArgs(), q->stream, lin);
        };
        CK(hipMemcpyAsync(q->x, x, sizeof(float) * d0.cols, hipMemcpyHostToDevice, q->stream));
        const float* nw = nullptr;
        Epi epi = EPI_STORE;
        if (variant & 1 || lin) {  // decode's gate/up launch: RMSNorm (unit weights), SwiGLU epilogue
            if (!q->nw) {
                std::vector<float> ones(d0.cols, 1.0f);
                q->nw = dalloc<float>(d0.cols);
                CK(hipMemcpy(q->nw, ones.data(), sizeof(float) * d0.cols, hipMemcpyHostToDevice));
            }
            nw = q->nw;
            epi = EPI_SWIGLU;
        }
        for (size_t c = 0; c < q->copies.size(); c++) mv(q->copies[c], nw, epi);  // warm: every copy once
        hipEvent_t a, b;
        CK(hipEventCreate(&a));
        CK(hipEventCreate(&b));
        CK(hipEventRecord(a, q->stream));
        for (int i = 0; i < iters; i++) mv(q->copies[(size_t)i % q->copies.size()], nw, epi);
        CK(hipEventRecord(b, q->stream));
        CK(hipEventSynchronize(b));
        float ms = 0.0f;
        CK(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        CK(hipGetLastError());
        *avg_us = 1000.0 * ms / iters;
        return 0;
    }, -1);
}

JYHIP_API jyhip_wmat* jyhip_wmat_upload(const jy_wmat* w, int n, int k, int copies) {
    return guarded([&]() -> jyhip_wmat* {
        if (!w || !w->data || n <= 0 || k <= 0) fail("bad weight matrix");
        if (!known_type(w->type)) fail("unsupported weight type");
        if (k % block_of(w->type)) fail("k is not a multiple of the type's block size");
        if ((w->type == JY_Q8_0 && matvec_lds_bytes(k, false) > matvec_lds_limit()) ||
            (block_of(w->type) == 256 && mv_kq_lds_bytes(k) > matvec_lds_limit()))
            fail("k too large for the decode matvec's LDS staging");
        if (copies <= 0) copies = 1;
        jyhip_wmat* h = new jyhip_wmat();
        h->n = n;
        h->k = k;
        jyhip_model holder;  // borrows put_w's bookkeeping
        try {
            int dev = 0;
            CK(hipGetDevice(&dev));
            init_device_kernels(dev);
            CK(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
            holder.stream = h->stream;
            uint8_t* staging = dalloc<uint8_t>(wbytes(w->type, n, k), false);
            try {
                for (int c = 0; c < copies; c++) h->copies.push_back(put_w(&holder, staging, *w, n, k));
            } catch (...) {
                dfree(staging);
                throw;
            }
            dfree(staging);
        } catch (...) {
            for (void* p : holder.owned) dfree(p);
            if (h->stream) (void)hipStreamDestroy(h->stream);
            delete h;
            throw;
        }
        h->owned.swap(holder.owned);
        holder.stream = nullptr;
        return h;
    }, nullptr);
}

JYHIP_API void jyhip_wmat_free(jyhip_wmat* h) {
    if (!h) return;
    (void)hipStreamSynchronize(h->stream);
    for (void* p : h->owned) dfree(p);
    (void)hipStreamDestroy(h->stream);
    delete h;
}

JYHIP_API int jyhip_wmat_matmul(jyhip_wmat* h, int m, const float* A, float* Cout) {
    return guarded([&]() {
        if (!h || !A || !Cout || m <= 0) fail("bad argument");
        const DevW& w = h->copies[0];
        float* a = dalloc<float>((size_t)m * h->k, false);
        float* c = dalloc<float>((size_t)m * h->n);
        try {
            CK(hipMemcpyAsync(a, A, sizeof(float) * (size_t)m * h->k, hipMemcpyHostToDevice, h->stream));
            if (m == 1)
                launch_mv(w, a, c, EPI_STORE, nullptr, h->stream);
            else
                launch_gemm(w, m, a, c, h->n, nullptr, EPI_STORE, h->stream);
            CK(hipGetLastError());
            CK(hipMemcpyAsync(Cout, c, sizeof(float) * (size_t)m * h->n, hipMemcpyDeviceToHost, h->stream));
            CK(hipStreamSynchronize(h->stream));
        } catch (...) {
            (void)hipStreamSynchronize(h->stream);
            dfree(a);
            dfree(c);
            throw;
        }
        dfree(a);
        dfree(c);
        return 0;
    }, -1);
}

JYHIP_API int jyhip_wmat_time(jyhip_wmat* h, const float* x, int iters, double* avg_us) {
    return guarded([&]() {
        if (!h || !x || !avg_us || iters <= 0) fail("bad argument");
        float* xd = dalloc<float>(h->k, false);
        float* yd = dalloc<float>(h->n);
        hipEvent_t a = nullptr, b = nullptr;
        try {
            CK(hipMemcpyAsync(xd, x, sizeof(float) * h->k, hipMemcpyHostToDevice, h->stream));
            for (const DevW& w : h->copies) launch_mv(w, xd, yd, EPI_STORE, nullptr, h->stream);  // warm
            CK(hipEventCreate(&a));
            CK(hipEventCreate(&b));
            CK(hipEventRecord(a, h->stream));
            for (int i = 0; i < iters; i++)
                launch_mv(h->copies[(size_t)i % h->copies.size()], xd, yd, EPI_STORE, nullptr, h->stream);
            CK(hipEventRecord(b, h->stream));
            CK(hipEventSynchronize(b));
            float ms = 0.0f;
            CK(hipEventElapsedTime(&ms, a, b));
            CK(hipGetLastError());
            *avg_us = 1000.0 * ms / iters;
        } catch (...) {
            (void)hipStreamSynchronize(h->stream);
            if (a) (void)hipEventDestroy(a);
            if (b) (void)hipEventDestroy(b);
            dfree(xd);
            dfree(yd);
            throw;
        }
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        dfree(xd);
        dfree(yd);
        return 0;
    }, -1);
}

}  // extern "C"
