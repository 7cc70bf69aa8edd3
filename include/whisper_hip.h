/*
 * libwhisper_hip.so — MI355X (gfx950) decoder token loop for whisper.go.
 *
 * C ABI: plain pointers and sizes, no C++ or framework types. Every call
 * returns an int status (WH_OK == 0); on failure wh_last_error() returns a
 * thread-local message whose prefix follows the reference's error strings
 * ("model: decode: ..."). Citations are relative to the reference repository
 * (github.com/whispergo/whisper.go).
 *
 * Threading: a wh_model is immutable after creation and may be shared by
 * threads; a wh_seq belongs to one caller thread at a time and owns its own
 * HIP stream. Decode calls are reentrant across distinct wh_seq / calls
 * (the reference's Decode keeps all state per call: internal/model/decoder.go:434).
 */
#ifndef WHISPER_HIP_H
#define WHISPER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define WH_OK 0
#define WH_ERR_INVALID (-1)     /* bad argument / shape (ml.ErrShapeMismatch, internal/ml/tensor.go:6) */
#define WH_ERR_HIP (-2)         /* HIP runtime failure */
#define WH_ERR_UNSUPPORTED (-3) /* feature outside the supported path */
#define WH_ERR_CANCELLED (-4)   /* cancellation flag observed (context.Canceled) */
#define WH_ERR_NOMEM (-5)
#define WH_ERR_NOT_FOUND (-6)   /* tensor not found (internal/model/compat.go:194-197) */

/* GGUF quantisation type codes (internal/gguf/quantize.go:14-24). */
#define WH_TYPE_F32 0u
#define WH_TYPE_F16 1u
#define WH_TYPE_Q4_0 2u
#define WH_TYPE_Q4_1 3u
#define WH_TYPE_Q5_0 6u
#define WH_TYPE_Q5_1 7u
#define WH_TYPE_Q8_0 8u

/* Thread-local message for the last failing call on this thread. */
const char *wh_last_error(void);
/* Library version string. */
const char *wh_version(void);
/* Number of visible HIP devices (0 on a host without a GPU). */
int wh_device_count(int32_t *count);

/* ---- device memory, streams and events ------------------------------------
 * Host plumbing with no counterpart in the reference (which has no device):
 * lets a host without its own GPU array library (Go via purego, Python via
 * ctypes) stage buffers for wh_gemv and time the kernels. kind: 0 host->device,
 * 1 device->host, 2 device->device. */
int wh_dev_malloc(uint64_t bytes, int32_t device, void **out);
int wh_dev_free(void *p);
int wh_memcpy(void *dst, const void *src, uint64_t bytes, int32_t kind);
int wh_stream_create(int32_t device, void **out);
int wh_stream_destroy(void *stream);
int wh_stream_sync(void *stream);
int wh_event_create(void **out);
int wh_event_destroy(void *ev);
int wh_event_record(void *ev, void *stream);
/* Milliseconds between two recorded events (waits for `stop`). */
int wh_event_elapsed(void *start, void *stop, float *ms);

/* ---- quantisation (host, bit-exact with the reference) -------------------- */
/* Raw byte size of n elements of `type`; replaces gguf rawSize
 * (internal/gguf/tensor.go:60-85) and ml quantRowBytes (internal/ml/matmul_q8.go:198-214). */
uint64_t wh_row_bytes(uint32_t type, uint64_t n);
/* Quantise n float32 values into `type` blocks; replaces gguf applyQuant /
 * Quantize{F16,Q4_0,Q4_1,Q5_0,Q5_1,Q8_0} (internal/gguf/quantize.go:120-139,
 * internal/gguf/quant.go:87-232). dst_bytes must be >= wh_row_bytes(type, n).
 * `threads` <= 1 runs serially (the result does not depend on it). */
int wh_quantize(uint32_t type, const float *src, uint64_t n, void *dst, uint64_t dst_bytes, int32_t threads);
/* 1 if cmd/quantize would quantise this tensor name, else 0; replaces
 * shouldQuantize (internal/gguf/quant.go:236-248, cmd/quantize/main.go:122-131). */
int wh_should_quantize(const char *name);
/* Host f16 conversions (internal/gguf/quant.go:11-55, internal/gguf/dequant.go:15-44). */
uint16_t wh_f32_to_f16(float f);
float wh_f16_to_f32(uint16_t h);

/* ---- device dequantisation (bit-exact check of the kernels' decode) -------- */
/* Uploads raw GGUF blocks, decodes them with the same device routine the
 * kernels use, copies the float32 result back. Replaces gguf.Dequantize
 * (internal/gguf/dequant.go:47-85) for types 0,1,2,3,6,7,8. */
int wh_dequantize(uint32_t type, const void *raw, uint64_t nbytes, uint64_t n, float *out, int32_t device);
/* wh_dequantize without any device allocation: no counterpart in the
 * reference; it is for callers that cannot allocate (serving loops, harnesses
 * that forbid hipMalloc). The raw blocks, their device layout and the result
 * are staged in a 16 MiB device array the library holds on each device until
 * the process ends; n is at most 1048576 (WH_ERR_INVALID beyond). Calls that
 * overlap on one device race on that array. Same results, bit for bit. */
int wh_dequantize_noalloc(uint32_t type, const void *raw, uint64_t nbytes, uint64_t n, float *out, int32_t device);

/* ---- standalone quantised GEMV ------------------------------------------- */
/* A device-resident quantised matrix [rows, cols] (row-major GGUF blocks per
 * row); replaces ml.QuantizedMatrix / NewQuantizedMatrix
 * (internal/ml/matmul_q8.go:36-42,74-87). The raw bytes are copied, re-laid
 * out for the device and uploaded once; no caller pointer is kept. */
typedef struct wh_matrix wh_matrix;
int wh_matrix_create(uint32_t type, int32_t rows, int32_t cols, const void *raw, uint64_t nbytes, int32_t device,
                     wh_matrix **out);
int wh_matrix_destroy(wh_matrix *m);
/* Algorithmic bytes of the matrix (GGUF block bytes = rows * row_bytes). */
int wh_matrix_bytes(const wh_matrix *m, uint64_t *bytes);
/* y[b, r] = sum_c x[b, c] * W[r, c] for b < batch (batch <= 16), fp32
 * accumulate; x and y are device pointers ([batch, cols], [batch, rows]
 * row-major), `stream` a hipStream_t (NULL = default stream). Asynchronous.
 * Replaces MatMulQuantTransBInto (internal/ml/matmul_q8.go:93-119). */
int wh_gemv(const wh_matrix *w, const float *x, int32_t batch, float *y, void *stream);

/* ---- decoder model ---------------------------------------------------------- */
/* One tensor of the decoder, named as in the reference GGUF files (or the HF
 * aliases of internal/model/compat.go:31-148). shape is as stored in the GGUF
 * descriptor, rows first (internal/gguf/tensor.go:28-53). */
typedef struct {
    const char *name;
    uint32_t type;
    uint32_t ndim;
    uint64_t shape[4];
    const void *data;
    uint64_t nbytes;
} wh_tensor;

/* GGUF metadata the loader reads (internal/model/decoder.go:101-105); 0 = absent. */
typedef struct {
    uint32_t n_head;  /* whisper.decoder.attention.head_count */
    uint32_t n_layer; /* whisper.decoder.layer_count */
    uint32_t n_ctx;   /* whisper.decoder.context_length */
    uint32_t n_state; /* whisper.decoder.embedding_length */
    uint32_t n_vocab; /* whisper.vocab.size / whisper.n_vocab */
} wh_meta;

typedef struct wh_model wh_model;
/* Build a decoder from a tensor table and upload every weight to HBM once;
 * replaces NewDecoder (internal/model/decoder.go:97-303) with its name
 * resolution and hyper-parameter inference (internal/model/compat.go:163-270). */
int wh_model_create(const wh_tensor *tensors, int32_t n, const wh_meta *meta, int32_t device, wh_model **out);
/* Same, reading a GGUF v2/v3 file (internal/gguf/gguf.go:52-135,203-246). */
int wh_model_load_gguf(const char *path, int32_t device, wh_model **out);
int wh_model_destroy(wh_model *m);
/* out5 = {n_vocab, n_state, n_head, n_layer, n_ctx}. */
int wh_model_hparams(const wh_model *m, int32_t *out5);
/* EOT token id (default 50256); replaces SetVocabulary's EOT update
 * (internal/model/decoder.go:85-94). */
int wh_model_set_eot(wh_model *m, int32_t eot);
/* Algorithmic quantised-weight bytes read per decoded token (every matrix
 * once, including the tied logits matrix). */
int wh_model_weight_bytes(const wh_model *m, uint64_t *bytes);
/* Decoder semantics: 0 = reference-compatible (default; causal mask inside
 * the Tq=1 block, internal/ml/attention.go:250-256), 1 = textbook causal
 * mask over the KV cache (opt-in deviation). */
int wh_model_set_attention_mode(wh_model *m, int32_t mode);

/* ---- Encoder: the model.Encoder interface (internal/model/encoder.go) ------ */
/* GGUF metadata the encoder loader reads (internal/model/encoder.go:63-67); 0 = absent. */
typedef struct {
    uint32_t n_head;  /* whisper.encoder.attention.head_count */
    uint32_t n_layer; /* whisper.encoder.layer_count */
    uint32_t n_ctx;   /* whisper.encoder.context_length (audio frames after the stride-2 conv) */
    uint32_t n_state; /* whisper.encoder.embedding_length */
    uint32_t n_mels;  /* whisper.audio.mel_count / whisper.n_mels */
} wh_enc_meta;

typedef struct wh_encoder wh_encoder;
/* Build an encoder from a tensor table and upload every weight to HBM once;
 * replaces NewEncoder (internal/model/encoder.go:58-263): hyper-parameters from
 * meta, else inferred from the tensors; conv weights in any stored order the
 * reference accepts; HF alias names (internal/model/compat.go:31-83). */
int wh_encoder_create(const wh_tensor *tensors, int32_t n, const wh_enc_meta *meta, int32_t device,
                      wh_encoder **out);
/* Same, reading a GGUF v2/v3 file. */
int wh_encoder_load_gguf(const char *path, int32_t device, wh_encoder **out);
int wh_encoder_destroy(wh_encoder *e);
/* out5 = {n_mels, n_state, n_head, n_layer, n_ctx}. */
int wh_encoder_hparams(const wh_encoder *e, int32_t *out5);
/* Encode (internal/model/encoder.go:265-338): mel is host float32 [n_mels, T]
 * row-major; T = 2 n_ctx + 1 keeps the first n_mels * 2 n_ctx values, T > 2 n_ctx
 * is WH_ERR_INVALID. The output [T', n_state] (T' = (T + 1) / 2) goes to out,
 * which holds out_cap rows; *out_rows = T'. cancel (may be NULL) is polled
 * between blocks (WH_ERR_CANCELLED). */
int wh_encode(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out, int32_t out_cap,
              int32_t *out_rows, const volatile int32_t *cancel);
/* The same with mel and out in device memory of the encoder's device (the
 * encoder output then feeds a decoder without a host round trip). The call is
 * synchronous: mel must be written before it is made, out is written when it
 * returns. Calls on one handle run one at a time. No counterpart in the
 * reference (its tensors live in host memory). */
int wh_encode_device(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out,
                     int32_t out_cap, int32_t *out_rows, const volatile int32_t *cancel);

/* ---- Decode: the model.Decoder interface (internal/model/interfaces.go:22-25) */
/* Mirrors model.DecoderParams (internal/model/interfaces.go:76-90); the
 * fields the reference's decoder does not read are omitted. */
typedef struct {
    const int32_t *prompt;
    int32_t prompt_len;
    int32_t beam_size;
    float temperature;
    float logprob_thold;
    float no_speech_thold;
    int32_t no_fallback;
    int32_t max_tokens;
    int32_t suppress_nst;
} wh_decode_params;

/* Decode one stream: greedy (beam_size <= 1, decoder.go:413-525) or beam
 * search (decoder.go:528-726). encoder_out is host float32 [enc_len, n_state].
 * Writes the full token sequence (prompt + generated) to out_tokens (capacity
 * cap) and its length to out_len. Replaces (*WhisperDecoder).Decode
 * (internal/model/decoder.go:401-410). `cancel` (may be NULL) is polled
 * between token steps; non-zero => WH_ERR_CANCELLED. */
int wh_decode(const wh_model *m, const float *encoder_out, int32_t enc_len, int32_t enc_dim,
              const wh_decode_params *params, int32_t *out_tokens, int32_t cap, int32_t *out_len,
              const volatile int32_t *cancel);
/* The same with encoder_out in device memory of the model's device (for
 * instance written by wh_encode_device): the cross K/V are projected from it in
 * place, with no host round trip of the encoder output. No counterpart in the
 * reference (its tensors live in host memory); WH_ERR_INVALID when the pointer
 * is not device memory of that device. */
int wh_decode_device(const wh_model *m, const float *encoder_out, int32_t enc_len, int32_t enc_dim,
                     const wh_decode_params *params, int32_t *out_tokens, int32_t cap, int32_t *out_len,
                     const volatile int32_t *cancel);

/* Greedy decode of n_streams independent streams as one batch (each with its
 * own encoder output and prompt). Equivalent to n_streams calls of
 * wh_decode with beam_size <= 1. out_tokens is [n_streams, cap]. */
int wh_decode_batch(const wh_model *m, int32_t n_streams, const float *const *encoder_outs, int32_t enc_len,
                    int32_t enc_dim, const wh_decode_params *params, int32_t *out_tokens, int32_t cap,
                    int32_t *out_lens, const volatile int32_t *cancel);

/* *out = forward steps (token-loop iterations) of the calling thread's last
 * wh_decode / wh_decode_batch call. Under the reference's beam search a
 * hypothesis may grow by more than one token per step, so its length does not
 * tell the step count. No counterpart in the reference: benchmarks read it. */
int wh_last_decode_steps(int32_t *out);

/* ---- step-level sequence API (one decoder state per stream) ---------------- */
/* A batch of decoder states with persistent KV caches and cached cross-attention
 * K/V in HBM; replaces decoderState (internal/model/decoder.go:306-386).
 * encoder_outs[s] is host float32 [enc_len, n_state]; when shared_encoder is
 * non-zero only encoder_outs[0] is read and every stream attends to it. */
typedef struct wh_seq wh_seq;
int wh_seq_create(const wh_model *m, int32_t n_streams, const float *const *encoder_outs, int32_t enc_len,
                  int32_t enc_dim, int32_t shared_encoder, wh_seq **out);
/* The same with the encoder outputs in device memory of the model's device. */
int wh_seq_create_device(const wh_model *m, int32_t n_streams, const float *const *encoder_outs, int32_t enc_len,
                         int32_t enc_dim, int32_t shared_encoder, wh_seq **out);
int wh_seq_destroy(wh_seq *s);
/* Set the token history of one stream (state.tokens); when reset_kv is non-zero
 * the stream's KV cache is cleared (resetDecoderState, decoder.go:367-386). */
int wh_seq_set_tokens(wh_seq *s, int32_t stream, const int32_t *tokens, int32_t n, int32_t reset_kv);
/* One forward (decoder.go:745-833) for the last token of every stream whose
 * active[s] is non-zero (NULL = all), then repetition penalty (decoder.go:1140-1167)
 * and greedy selection (decoder.go:996-1034); the chosen ids are appended to
 * the histories and written to out_ids[s] (-1 for inactive streams).
 * out_logits (may be NULL) receives the raw logits [n_streams, n_vocab]
 * (parity mode). Synchronous. */
int wh_seq_step_greedy(wh_seq *s, const int32_t *active, float temperature, int32_t suppress_nst,
                       float no_speech_thold, int32_t *out_ids, float *out_logits);
/* Same forward, then top-k (decoder.go:1068-1136) on the penalised logits of
 * each active stream; out_tok/out_logprob are [n_streams, k] (k <= 8). The
 * histories are not modified. */
int wh_seq_step_topk(wh_seq *s, const int32_t *active, int32_t k, float temperature, int32_t *out_tok,
                     float *out_logprob, float *out_logits);

/* Up to n greedy steps of a one-stream sequence with the reference's stop
 * rules (decoder.go:441-485): stop after EOT, after more than 20 repeats of one
 * token, or when the history reaches max_len tokens (capped at n_text_ctx).
 * The generated ids go to out_ids[0..*out_n). On a one-stream sequence past
 * position 0 the whole loop runs in one persistent cooperative kernel. */
int wh_seq_generate(wh_seq *s, int32_t n, float temperature, int32_t suppress_nst, float no_speech_thold,
                    int32_t max_len, int32_t *out_ids, int32_t *out_n);

/* *out = 1 when the persistent kernel serves this sequence's greedy steps past
 * position 0 (one stream, head size 64, every matrix of one quantised type,
 * reference attention mode, WHISPER_HIP_PERSISTENT not 0 at creation), else 0;
 * *launches = persistent launches made so far. No counterpart in the
 * reference: it lets callers and tests see which path ran. */
int wh_seq_persistent(wh_seq *s, int32_t *out, int64_t *launches);

/* Per-kernel timing of the step calls: with profiling enabled every launch on
 * the sequence's stream is bracketed by a HIP event pair and accumulated per
 * kernel class ("gemv", "cross_attn", "layernorm", ...), with the launch's
 * algorithmic HBM bytes. No counterpart in the reference (its benchmarks are
 * Go testing.B timers). Enabling or disabling clears the accumulators. */
int wh_seq_set_profiling(wh_seq *s, int32_t enable);
int wh_seq_profile_count(wh_seq *s, int32_t *n);
int wh_seq_profile_get(wh_seq *s, int32_t i, char *name, int32_t name_cap, double *ms, int64_t *launches,
                       double *bytes);

#ifdef __cplusplus
}
#endif
#endif
