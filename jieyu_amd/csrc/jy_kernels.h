// jy_kernels.h — host-side launchers for the decode-path HIP kernels.
//
// Device data layouts (resident in HBM for the life of a model):
//  Q8_0 weight matrices: row groups of 4 x chunks of 8 blocks (jy_layout.h).
//  f32 / f16 weight matrices: jieyu's [in][out] (libs/matmul_libs/matmul.h:7) as
//    ceil(N/64) panels of [K][64] row-major, columns past N zero.
//  KV cache: K and V int8 [L][nkv][max_seq][hd], scales fp32 [L][nkv][max_seq]
//    (head-major, so one head's keys are contiguous; jieyu keeps [L][pos][nkv][hd],
//    libs/date_libs/date.h:89-147 — jyhip_kv_read/_write convert).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jy {

enum Epi { EPI_STORE = 0, EPI_BIAS = 1, EPI_RESID = 2, EPI_SWIGLU = 3, EPI_ROPE = 4, EPI_ARGMAX = 5 };

struct Q8Dev {
    uint8_t* qs = nullptr;
    uint16_t* d = nullptr;
    int rows = 0, cols = 0, nb = 0, nch = 0, nbp = 0, rows_pad = 0;
    int nchp = 0;  // chunks stored per row group: nch rounded up to a multiple of 2*U
    int U = 0;     // decode matvec register-buffer depth (chunks per buffer, two buffers)
};

// A Q8_0 matrix as the matrix-core prompt GEMM reads it (jy_gemm_mfma.hip): per tile of
// 16 rows and block of 32 weights, 512 bytes in MFMA B-operand lane order (q), and the
// block scales as fp32, four blocks of a row together (d).  Rows past `rows` are zero.
struct Q8MfmaDev {
    int8_t* q = nullptr;  // [tiles][nb][64 lanes][8]
    float* d = nullptr;   // [tiles][nb4][16 rows][4]
    int rows = 0, cols = 0, nb = 0, nb4 = 0, tiles = 0;
};

// A Q4_K / Q5_K / Q6_K matrix of rows x cols (cols a multiple of 256), repacked so
// that one 256-weight super-block of four rows is read by one wave, thread
// t = ri*16 + g (row ri of the group, lane pair g) owning weights 32c + 2g + u
// (u = 0, 1) of the eight 32-weight steps c, as in the Q8_0 layout.  Chunk =
// (row group, super-block), chunk index (R >> 2) * nsb + sb.  A thread's 16 weights
// are addressed as (target T, byte k): T = 2*(c >> 2) + u, k = c & 3, so that each
// of its four 32-bit nibble words (T) holds one weight per byte after a mask.
//   nib : 512 B per chunk, 8 B per thread: nibble 2c + u (c = 0..7) is the low 4
//         bits of weight (c, u), so word 0 holds c = 0..3 and word 1 c = 4..7
//   hi  : Q5_K 2 B per thread, bit 4T + k = the fifth bit of weight (T, k);
//         Q6_K 4 B per thread, bits 8k + 2T, 8k + 2T + 1 = the top two bits
//   hdr : 16 B per row: Q4_K / Q5_K the eight 6-bit scales then the eight 6-bit
//         mins, one per byte; Q6_K the int8 scale of each step c for the row's
//         first 16 weights (bytes 0..7) and last 16 (bytes 8..15)
//   dm  : 4 B per row: fp16 d (and Q4_K / Q5_K dmin in the high half)
// Bytes per 256 weights: 148 / 180 / 212 (GGML's 144 / 176 / 210 with the scales
// unpacked).
struct KQDev {
    int type = 0;  // JY_Q4_K | JY_Q5_K | JY_Q6_K
    int rows = 0, cols = 0, nsb = 0, groups = 0;
    uint8_t* nib = nullptr;
    uint8_t* hi = nullptr;
    uint8_t* hdr = nullptr;
    uint32_t* dm = nullptr;
};

// One weight matrix of any bound type (jieyu's WMat, libs/date_libs/wmat.h:32-44):
// JY_F32 / JY_F16 [in][out] dense in 64-column panels (the embedding table excepted:
// [vocab][hidden] rows), JY_Q8_0 in the Q8 layout, k-quants in KQDev.
struct DevW {
    int type = 0;
    int in = 0, out = 0;
    const void* dense = nullptr;
    Q8Dev q8;
    KQDev kq;
};

struct KVDev {
    int8_t* k = nullptr;
    int8_t* v = nullptr;
    float* ks = nullptr;
    float* vs = nullptr;
    int num_layers = 0, max_seq = 0, nkv = 0, hd = 0;
};

// Epilogue arguments of the decode matvec.
struct MvArgs {
    const float* aux = nullptr;      // bias (EPI_BIAS / EPI_ROPE) or nothing
    const int* state = nullptr;      // [0] = sequence length (position = state[0]-1), [1] = stop flag
    int pos0 = 0;                    // EPI_ROPE position when state is null
    const float* cos_t = nullptr;    // EPI_ROPE tables [max_seq][hd/2]
    const float* sin_t = nullptr;
    int nh = 0, nkv = 0, hd = 0;     // EPI_ROPE: rows [0, nh*hd) are q, then k, then v
    int* ids = nullptr;              // EPI_ARGMAX: token ids (next id goes to ids[state[0]])
    int* mstate = nullptr;           // EPI_ARGMAX: mutable state
    const int* eos = nullptr;
    int neos = 0;
    float* part_val = nullptr;       // EPI_ARGMAX: per-workgroup partial maxima (argmax_partials(rows) each)
    int* part_idx = nullptr;
};

size_t q8_qs_bytes(int rows, int cols);
size_t q8_d_bytes(int rows, int cols);
Q8Dev q8_shape(int rows, int cols);

// Once per device, before any launch: raise the dynamic LDS limit of the kernels
// that stage a full activation vector.
hipError_t kernels_init();
hipError_t gemm_mfma_init();

// src: jieyu Q8_0 rows [rows][cols/32] x 34 B (device copy).  Source row r lands
// in destination row row_base + r*row_stride.
void launch_repack_q8(const uint8_t* src, int rows, int cols, const Q8Dev& dst, int row_base, int row_stride,
                      hipStream_t st);

// Embedding rows.  ids_dev[id_index0 + i] (or, when state != null, ids_dev[state[0]-1])
void launch_embed(const Q8Dev* q8, const float* f32, int hidden, const int* ids_dev, int id_index0,
                  const int* state, int seq, float* X, hipStream_t st);

// RMSNorm (eps 1e-5) of `rows` rows of n floats
void launch_rmsnorm(const float* X, float* Y, const float* w, int n, int rows, hipStream_t st);

// y = W x for one token in the reference's 32-lane order; when norm_w != null the
// kernel first applies RMSNorm (eps 1e-5) to x with those weights, or with norm_linear
// (the tolerance mode) scales each finished dot by the norm factor instead.  EPI_ARGMAX
// also launches the one-workgroup pick over the per-workgroup maxima.
void launch_matvec_q8(const Q8Dev& W, const float* x, const float* norm_w, float* out, Epi epi, const MvArgs& a,
                      hipStream_t st, bool norm_linear = false);
// the same y = W x with each row's dot split over waves in a free order (the tolerance
// mode), RMSNorm applied after the dot by linearity; same epilogues
void launch_matvec_q8_split(const Q8Dev& W, const float* x, const float* norm_w, float* out, Epi epi,
                            const MvArgs& a, hipStream_t st);
// workgroups (argmax partials) of a split EPI_ARGMAX launch over `rows` rows
int split_argmax_partials(int rows);
// LDS the Q8 matvec takes for rows of `cols` (staged x, and the norm weights with
// NORM), and what one workgroup may take (valid after kernels_init)
size_t matvec_lds_bytes(int cols, bool norm);
size_t matvec_lds_limit();
// dense [K][N] matvec over the 64-column panel layout (f32, or f16 converted exactly),
// fma chain over k per output column: EPI_STORE / EPI_BIAS / EPI_RESID, or
// EPI_SWIGLU: out = silu(aux) * (W x)
void launch_matvec_f32(const float* B, int K, int N, const float* x, float* out, const float* aux, Epi epi,
                       hipStream_t st);
void launch_matvec_f16(const uint16_t* B, int K, int N, const float* x, float* out, const float* aux, Epi epi,
                       hipStream_t st);
// prefill GEMMs, C[m][N] (+ epilogue: EPI_STORE / EPI_BIAS / EPI_RESID)
void launch_gemm_q8(const Q8Dev& W, int m, const float* A, float* C, const float* aux, Epi epi, hipStream_t st);
// the matrix-core form (jy_gemm_mfma.hip): the copy of W it reads (built once), the split
// of the activations A [m][K] into fp16 high / low parts over mfma_rows_padded(m) rows
// (rows past m zero) with each row's power-of-two unscale, and C[m][ldc] (+ epilogue:
// EPI_STORE / EPI_BIAS / EPI_RESID) from them
void launch_mfma_repack(const Q8Dev& W, const Q8MfmaDev& M, hipStream_t st);
int mfma_rows_padded(int m);
void launch_mfma_split(const float* A, int m, int mp, int K, _Float16* hi, _Float16* lo, float* unscale,
                       hipStream_t st);
// the RMSNorm of X's rows (rmsnorm_kernel's arithmetic) and the split above in one kernel;
// with kz > 1 (only where mfma_norm_split_takes_parts(K)) X += the kz partials in kp first
// ([kz][m][K], a deferred residual GEMM split over K), written back to X
bool mfma_norm_split_takes_parts(int K);
void launch_mfma_norm_split(float* X, int m, int mp, int K, const float* nw, _Float16* hi, _Float16* lo,
                            float* unscale, hipStream_t st, const float* kp = nullptr, int kz = 0);
// (kpart: kpart_n floats for the partial sums of a GEMM split over K, or nullptr: no split.
// With defer, a split GEMM leaves its sum to the caller: the return value is then the
// number of partials in kpart ([Z][m][W.rows]), 0 when C holds the result)
int launch_gemm_q8_mfma(const Q8MfmaDev& W, int m, const _Float16* hi, const _Float16* lo, const float* unscale,
                        float* C, int ldc, const float* aux, Epi epi, hipStream_t st, float* kpart = nullptr,
                        size_t kpart_n = 0, bool defer = false);
// the deferred sum: C (+)= the Z partials [Z][m][N], with the epilogue
void launch_gemm_ksum(const float* kpart, int Z, int m, int N, float* C, int ldc, const float* aux, Epi epi,
                      hipStream_t st);
// the K slices launch_gemm_q8_mfma takes for these rows, and the partial floats they need
int gemm_q8_mfma_ksplit(const Q8MfmaDev& W, int m, Epi epi);
size_t gemm_q8_mfma_kpart_floats(const Q8MfmaDev& W, int m, Epi epi);
void launch_gemm_f32(const float* B, int K, int N, int m, const float* A, float* C, const float* aux, Epi epi,
                     hipStream_t st);
// h[i][j] = silu(gu[i][2j]) * gu[i][2j+1]  (or silu(g) * u with separate buffers)
void launch_silu_mul(const float* g, const float* u, int interleaved, int m, int F, float* h, hipStream_t st);

// RoPE on q and k of every row, K/V int8 packing into the cache of `layer`, Q int8.
// qkv: [seq][q_dim + 2*kv_dim] (read only).  Position start_pos + row, or state[0]-1 when
// state != null (a one-row decode step).  kz > 1: the rows are instead the sums of the kz
// partials in kp ([kz][seq][q_dim + 2*kv_dim], launch_gemm_q8_mfma's deferred split), plus
// bias when given.
void launch_rope_pack(const float* qkv, int seq, int start_pos, const int* state, int nh, int nkv, int hd,
                      const float* cos_t, const float* sin_t, const KVDev& kv, int layer, int8_t* q8, float* qsc,
                      hipStream_t st, const float* kp = nullptr, int kz = 0, const float* bias = nullptr);
hipError_t rope_pack_init();

struct AttnArgs {
    // fused (decode): q, k, v rows of the token from qkv (already roped); the kernel
    // quantizes them and appends K/V at position state[0]-1.  Otherwise q8/qsc come
    // from launch_rope_pack and every key is already in the cache.
    bool fused = false;
    const float* qkv = nullptr;
    const int8_t* q8 = nullptr;
    const float* qsc = nullptr;
    int row0 = 0, nrows = 1, start_pos = 0;
    const int* state = nullptr;
    int nh = 0, nkv = 0, hd = 0;
    KVDev kv;
    int layer = 0;
    float* scratch = nullptr;        // scores between the two attention kernels: nrows*nh*max_keys floats
    int max_keys = 0;
    float* out = nullptr;            // [rows][nh*hd]
    // with state: every position the launch will be replayed at attends at most
    // att_short_keys() keys (then one kernel computes the scores too)
    bool short_ctx = false;
};
void launch_attention(const AttnArgs& a, hipStream_t st);
int att_short_keys();
// decode attention split over the keys (jy_attention_split.hip): one token row (fused
// q/k/v, nrows 1), `ns` slices (attn_split_slices of the longest length the launch may
// see); part: attn_split_part_floats(nh, hd, ns) floats
bool attn_split_supported(int nh, int nkv, int hd);
int attn_split_slices(int keys);
size_t attn_split_part_floats(int nh, int hd, int ns);
void launch_attention_split(const AttnArgs& a, float* part, int ns, hipStream_t st);
// the same token row attending at most att_whole_keys() keys: one kernel, one workgroup per
// (kv head, 16 output dims) over all the keys, output to a.out
int att_whole_keys();
void launch_attention_whole(const AttnArgs& a, hipStream_t st);
// prompt rows in the same arithmetic (q8 / qsc from launch_rope_pack, keys in the cache,
// a.nrows rows from a.row0): one workgroup per (kv head, row), output to a.out
void launch_attention_prefill_split(const AttnArgs& a, hipStream_t st);

// ---- the persistent decode kernel (jy_decode_persist.hip), tolerance mode
// One Q8_0 matrix as the persistent kernel streams it: its layout and the plan of its
// wave streams (SK waves per row group, U-chunk buffers, `per` passes per workgroup).
struct PMat {
    const uint8_t* qs = nullptr;
    const uint16_t* d = nullptr;
    int rows = 0, cols = 0, nch = 0, nchp = 0, nbp = 0;
    int SK = 1, U = 1, per = 0;
};
struct PLayer {
    PMat qkv, o, gu, down;
    const float* rms1 = nullptr;
    const float* rms2 = nullptr;
    const float* bqkv = nullptr;
};
struct PersistArgs {
    const PLayer* layers = nullptr;  // device array [L]
    int L = 0, H = 0, F = 0;
    PMat lm;
    const float* final_rms = nullptr;
    const float* cos_t = nullptr;
    const float* sin_t = nullptr;
    AttnArgs att;  // one fused decode row: qkv, kv, state or start_pos, out (the attention output)
    float* X = nullptr;
    float* qkv = nullptr;
    float* h = nullptr;
    float* part = nullptr;  // attention slices: attn_split_part_floats(nh, hd, ns)
    int ns = 1;
    unsigned* flags = nullptr;  // [workgroups] barrier flags, then [nkv] slice counters: zero at launch
    unsigned* acnt = nullptr;
    int* err = nullptr;         // set when a barrier wait gave up
    float* layer_x = nullptr;   // optional [L][H]: X after every layer
    int head = 0;               // 1: final RMSNorm + lm_head + greedy pick into ids / mstate
    float* logits = nullptr;
    float* part_val = nullptr;  // [workgroups]
    int* part_idx = nullptr;
    int* ids = nullptr;
    int* mstate = nullptr;
    const int* eos = nullptr;
    int neos = 0;
};
bool persist_supported(int nh, int nkv, int hd);
int persist_workgroups();
int persist_slices(int nkv, int max_keys);
size_t persist_lds_bytes(int max_nbp, int hd);
bool persist_resident(int hd, size_t lds);
void persist_plan(PMat& M, int nwg);
void launch_decode_persist(const PersistArgs& A, size_t lds, hipStream_t st);

// greedy next token (with repetition penalty): ids[state[0]] = argmax; state[0]++
void launch_argmax(const float* logits, int V, int* ids, int* state, const int* eos, int neos, float rep_penalty,
                   int prompt_len, hipStream_t st);

// reference-layout <-> device-layout KV rows for one layer
void launch_kv_import(const int8_t* k_ref, const float* ks_ref, const int8_t* v_ref, const float* vs_ref,
                      int pos0, int npos, const KVDev& kv, int layer, hipStream_t st);
void launch_kv_export(int8_t* k_ref, float* ks_ref, int8_t* v_ref, float* vs_ref, int pos0, int npos,
                      const KVDev& kv, int layer, hipStream_t st);

// zeros over `bytes` (a multiple of 16, 16-byte aligned) of device memory, by a kernel
void launch_zero_fill(void* p, size_t bytes, hipStream_t st);

// argmax partials workspace for an EPI_ARGMAX matvec of `rows` rows
int argmax_partials(int rows);

// ---- weights of any type (jy_quant.hip)
KQDev kq_shape(int type, int rows, int cols);
size_t kq_bytes(const KQDev& w, int part);  // part 0 nib, 1 hi, 2 hdr, 3 dm
// src: GGML blocks [rows][cols/256] (device copy) -> dst
void launch_repack_kq(const uint8_t* src, const KQDev& dst, hipStream_t st);
// y = W x for one token, in the reference's order for W's type (32-lane dot for
// quantized rows, fma chain over k for dense [in][out]); EPI_STORE / EPI_BIAS /
// EPI_RESID
void launch_mv(const DevW& W, const float* x, float* out, Epi epi, const float* aux, hipStream_t st);
// C[i][j] (row stride ldc) for m > 1 rows: the generic quantized path (product and
// sum rounded apart, k ascending) or the dense fma chain
void launch_gemm(const DevW& W, int m, const float* A, float* C, int ldc, const float* aux, Epi epi,
                 hipStream_t st);
// embedding rows of any type (wmat_row, libs/model_libs/wmat_kernel.h:18-29)
void launch_embed_w(const DevW& E, int hidden, const int* ids_dev, int id_index0, const int* state, int seq,
                    float* X, hipStream_t st);
size_t mv_kq_lds_bytes(int cols);
hipError_t quant_init();

}  // namespace jy
