// Internal declarations shared by the host (.cpp) and device (.hip) sources of
// libwhisper_hip.so. Not part of the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/whisper_hip.h"

namespace wh {

// ---- errors -----------------------------------------------------------------
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
#define WH_HIP(call)                                                                         \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess)                                                                \
            return ::wh::fail(WH_ERR_HIP, std::string("hip: ") + #call + ": " + hipGetErrorString(e_)); \
    } while (0)

// ---- device matrix layout ------------------------------------------------------
// A GGUF-block matrix [rows, cols] re-laid out for coalesced 128-bit streaming:
// quants and per-block scale words live in separate row-major planes so every
// lane's block payload is 16-byte aligned. Values are bit-identical to the
// GGUF blocks (the same f16 words, nibbles and high bits).
//   F32 (F16 is widened to F32 exactly at upload):  f32  [rows][nb*32]
//   Q8_0: qs int8 [rows][nb*32]   sc f16   [rows][nb]
//   Q4_0: qs u8   [rows][nb*16]   sc f16   [rows][nb]
//   Q4_1: qs u8   [rows][nb*16]   sc f16x2 [rows][nb]  (d low, m high)
//   Q5_0: qs u8   [rows][nb*16]   qh u32   [rows][nb]   sc f16   [rows][nb]
//   Q5_1: qs u8   [rows][nb*16]   qh u32   [rows][nb]   sc f16x2 [rows][nb]
// Padding of the tail block (cols % 32 != 0) is whatever the GGUF tail block
// holds; kernels mask x beyond cols.
struct DevMat {
    uint32_t type = 0;
    int32_t rows = 0, cols = 0, nb = 0;
    void *qs = nullptr;       // quants (or f32 data)
    void *sc = nullptr;       // scale words (uint16 or uint32)
    uint32_t *qh = nullptr;   // Q5 high bits
    void *alloc = nullptr;    // single device allocation holding all planes
    uint64_t algo_bytes = 0;  // GGUF bytes (rows * row_bytes)
    uint64_t dev_bytes = 0;
};

uint64_t gguf_row_bytes(uint32_t type, uint64_t n);
bool is_quant_type(uint32_t type);
uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);
int quantize(uint32_t type, const float *src, uint64_t n, uint8_t *dst, uint64_t dst_bytes, int threads);
int should_quantize(const char *name);
// Host dequantisation of raw GGUF data (internal/gguf/dequant.go:47-201).
int dequantize_host(uint32_t type, const uint8_t *raw, uint64_t n, float *out);
// Size the device planes for a [rows, cols] matrix of `type`, then scatter the
// raw GGUF rows (of src_type) into them and upload.
int devmat_plan(DevMat &m, uint32_t type, int32_t rows, int32_t cols);
int devmat_upload_typed(DevMat &m, uint32_t src_type, const uint8_t *raw, uint64_t nbytes);
void devmat_free(DevMat &m);

// ---- model ------------------------------------------------------------------------
struct Layer {
    float *ln1w, *ln1b, *sqb, *svb, *sob, *ln2w, *ln2b, *cqb, *cvb, *cob, *ln3w, *ln3b, *fc1b, *fc2b;
    DevMat sq, sk, sv, so, cq, ck, cv, co, fc1, fc2;
    // q, k, v stacked as one [3d, d] matrix when they share a quantised type;
    // sq/sk/sv are then views into its planes (alloc == nullptr)
    DevMat sqkv;
    // LayerNorm folded into the rows that read its output (persistent decode):
    // W·LN(x) = rsd * (W·(w*x) - mean * (W·w)) + (W·b + bias), so per row W·w
    // (cqc: cross query rows with ln2; f1c: fc1 rows with ln3) and W·b + bias
    // (cqe, f1e). Null when the matrices are not quantised.
    float *cqc = nullptr, *cqe = nullptr, *f1c = nullptr, *f1e = nullptr;
};
// Stack same-type matrices with equal column counts into one allocation; the
// parts become views into it.
int devmat_stack(std::vector<DevMat *> parts, DevMat &out);

}  // namespace wh

struct wh_model {
    int32_t device = 0;
    int32_t n_vocab = 0, n_state = 0, n_head = 0, n_layer = 0, n_ctx = 0;
    int32_t eot = 50256;
    int32_t attn_mode = 0;  // 0 reference-compatible, 1 textbook causal
    wh::DevMat tok;         // token embedding [n_vocab, n_state] (tied logits matrix)
    float *pos = nullptr;   // positional embedding [n_ctx, n_state]
    float *lnw = nullptr, *lnb = nullptr;
    std::vector<wh::Layer> layers;
    void *vec_alloc = nullptr;  // one allocation for every float vector
    void *fold_alloc = nullptr;  // the folded LayerNorm row constants of every layer
    uint64_t weight_bytes = 0;
};

struct wh_matrix {
    wh::DevMat m;
    int32_t device = 0;
};

namespace wh {

// ---- kernel launchers (wh_kernels.hip) --------------------------------------------
struct GemvOut {
    float *y = nullptr;        // [batch, ldy]
    int32_t ldy = 0;
    const float *bias = nullptr;
    const float *res = nullptr;  // y = res + (dot + bias)  (res may alias y)
    int32_t ldres = 0;
    int32_t gelu = 0;            // y = gelu(dot + bias)
};
struct GemvIn {
    const float *x = nullptr;  // [batch, ldx]
    int32_t ldx = 0;
};
// Workspace of the batched matrix-core GEMV's split-K path, owned by one stream of
// launches: partial tiles of at most `tiles` 16-row tiles as {launch number, value}
// pairs (zero when allocated) and one arrival counter per tile (zero when
// allocated; the kernel leaves it zero). `seq` numbers the launches.
constexpr int GEMVM_MAX_SPLIT = 4;
#ifndef GEMVM_SPLIT_TILES
#define GEMVM_SPLIT_TILES 320  // row tiles a sequence's workspace holds
#endif
struct GemvWork {
    uint64_t *part = nullptr;  // tiles * GEMVM_MAX_SPLIT * 256 pairs
    uint32_t *cnt = nullptr;   // tiles counters
    int tiles = 0;
    uint32_t seq = 0;
};
// Up to 3 matrices of the same type in one launch (e.g. q,k,v). `work` (optional)
// lets batches of 6..16 rows split K over more workgroups.
int launch_gemv(const DevMat *const *mats, const GemvIn *in, const GemvOut *out, int nmat, int batch,
                hipStream_t st, GemvWork *work = nullptr);
int launch_dequant_rows(const DevMat &m, int32_t row0, int32_t nrows, float *out, hipStream_t st);
// wh_dequantize with every staging buffer in a file-scope device array (wh_noalloc.hip).
int dequantize_noalloc(uint32_t type, const void *raw, uint64_t nbytes, uint64_t n, float *out, int32_t device);

struct SeqDev;  // defined in wh_seq.cpp
int launch_embed(const wh_model &m, const int32_t *tok, const int32_t *pos, const int32_t *active, float *x,
                 int S, hipStream_t st);
int launch_layernorm(const float *x, const float *w, const float *b, float *y, int S, int d, hipStream_t st);
int launch_self_attn(const float *q, const float *k, const float *v, float *kv_layer, size_t kv_stream_stride,
                     const int32_t *pos, const int32_t *active, float *out, int S, int H, int hd, int ctx,
                     int mode, hipStream_t st);
struct CrossBufs {
    float *scores;     // [S][H][enc_len]
    float *cmax;       // [S][H][C]
    uint64_t *pvt;     // [S][H][C][65] {launch number, value}: a chunk's weights . V and its weight sum
    uint32_t *cnt;     // [S][H] chunks arrived, zero between launches
    uint32_t seq;      // launch number of the last head-size-64 launch
    int chunks;
    int chunk_len;
};
int launch_cross_attn(const float *q, const float *const *kbase, const float *const *vbase, const int32_t *active,
                      float *out, int S, int H, int hd, int enc_len, CrossBufs &b, hipStream_t st);
// out[T, rows] = enc[T, cols] . w^T (+ bias); gelu: gelu of that; res: res + that.
int launch_cross_gemm(const DevMat &w, const float *enc, int enc_len, const float *bias, float *out,
                      hipStream_t st, int gelu = 0, const float *res = nullptr);
// The same for n (1..3) matrices over the same frames in one launch when they
// share type and row length (otherwise one launch each): out[i] = enc . ws[i]^T + bias[i].
int launch_cross_gemm_n(const DevMat *const *ws, int n, const float *enc, int enc_len, const float *const *bias,
                        float *const *out, hipStream_t st, int gelu = 0, const float *res = nullptr);
// encoder kernels (wh_encoder.hip)
int launch_im2col(const float *in, int64_t sc, int64_t st, int cin, int tin, int stride, int tout, int K, float *out,
                  hipStream_t s);
int launch_gelu_add(float *x, const float *pos, int64_t n, hipStream_t s);
int launch_enc_attn(const float *Q, const float *K, const float *V, int T, int d, int H, float *out, hipStream_t s);
// Load the code objects of wh_encoder.hip and wh_kernels.hip ahead of their first launch.
int warm_encoder_kernels();
int warm_kernels();
struct SampleBufs {
    float *cur;          // [S][V] penalised logits
    float *part_val;     // [S][P]
    int32_t *part_idx;   // [S][P]
    float *part_val2;    // [S][P] best excluding eot
    int32_t *part_idx2;
    int parts;
    // per-stream sampling parameters (DecoderParams of each stream)
    float *inv_temp;     // [S] 1 / temperature
    int32_t *supp;       // [S] SuppressNST
    float *nst;          // [S] NoSpeechThold
};
int launch_penalty_argmax(const float *logits, const int32_t *hist, const int32_t *hist_len, int hist_cap,
                          const int32_t *active, int S, int V, int eot, const SampleBufs &b, hipStream_t st);
int launch_argmax_final(const SampleBufs &b, const float *cur, int S, int V, int eot, const int32_t *active,
                        int32_t *hist, int32_t *hist_len, int hist_cap, int32_t *tok, int32_t *pos, int32_t *out_ids,
                        hipStream_t st);
// Exact top-k of rows whose k_topk result has ties (the reference's replace-min scan).
int launch_topk_ties(const float *cur, const int32_t *active, int S, int V, int k, int kk, float inv_temp,
                     const float *logz, int32_t *tok, float *lp, hipStream_t st);
// One beam step's candidate ranking (Go's sort.Slice order), prune and in-place
// reuse of the beam objects' histories on the device. `step` is recorded in
// stop[3] when the step stops the search or finds a position past the context.
int launch_beam_select(const int32_t *ttok, const float *tlp, int k, int kk, int32_t *hist, int32_t *len,
                       int32_t *gcap, int cap, float *score, int32_t *order, int32_t *nbeams, int32_t *active,
                       int32_t *tok, int32_t *pos, int32_t *stop, const float *powtab, int bs, int eot, int n_ctx,
                       int step, hipStream_t st);
// top-k scratch: TOPK_ROWS_MAX x TOPK_PARTS partitions x (2 + 2 * 8) floats
constexpr int TOPK_ROWS_MAX = 16, TOPK_PARTS = 32, TOPK_SCRATCH_FLOATS = TOPK_ROWS_MAX * TOPK_PARTS * 18;
int launch_topk(const float *cur, const int32_t *active, int S, int V, int k, float inv_temp, int32_t *out_tok,
                float *out_lp, float *out_logz, float *part, hipStream_t st);

}  // namespace wh
