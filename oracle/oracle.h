/*
 * CPU oracle for the whisper.go decoder token loop.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * algorithm (wxcdart/whisper.go, Go module github.com/whispergo/whisper.go),
 * used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg to
 * check and time against. The product (libwhisper_hip.so) never links, loads or
 * calls it.
 *
 * Each function cites the reference file:line it restates. Float arithmetic
 * is float32 with no FMA contraction (Go on amd64, GOAMD64=v1, does not fuse),
 * compiled with -ffp-contract=off.
 *
 * Parity pinning (what checks each part, see tests/test_oracle_*.py):
 *   f16<->f32, dequant     : reference KATs (gguf_test.go:155-309) + exhaustive
 *                            f16 decode vs numpy + closed form per format.
 *   quantizers             : closed-form invariants, round-trip bounds
 *                            (quant_test.go:11-127), brute force on tiny blocks.
 *   dot / GEMV             : float64 brute force, matmul_q8_test.go tolerances.
 *   LN / GELU / softmax /
 *   SDPA                   : ops_test.go:223-437, attention_test.go:9-60,
 *                            textbook closed forms (math.exp / math.tanh).
 *   penalty/argmax/top-k   : decoder_bench_test.go:65-73 logits pattern,
 *                            brute-force sort.
 *   decoder loop           : decoder_test.go fixture behaviour + invariants
 *                            (P1/P2 self-attn collapse, P3 cross addressing).
 *   beam prune             : Go's sort.Slice restated (pdqsort_func): sortedness
 *                            and permutation by brute force, insertion-sort
 *                            stability up to 12 items, hand-traced tie orders;
 *                            in-place beam reuse: hand-derived histories.
 *   Parity unpinned        : end-to-end logits/tokens of the reference on any
 *                            configuration (no golden logits exist and the Go
 *                            toolchain is absent), sgemm summation order
 *                            (gonum / OpenBLAS), and sort.Slice tie orders
 *                            beyond the hand-traced cases.
 */
#ifndef WHISPER_ORACLE_H
#define WHISPER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions -------------------------------------------------- */
float or_f16_to_f32(uint16_t h);          /* gguf/dequant.go:15-44 */
uint16_t or_f32_to_f16(float f);          /* gguf/quant.go:11-55 */

/* ---- block formats ------------------------------------------------------- */
size_t or_row_bytes(uint32_t type, size_t n);                         /* gguf/tensor.go:60-85 */
int or_dequantize(const uint8_t *raw, uint32_t type, size_t n, float *out); /* gguf/dequant.go:47-201 */
size_t or_quantize(const float *src, size_t n, uint32_t type, uint8_t *dst); /* gguf/quant.go:87-232 */
int or_should_quantize(const char *name);                           /* gguf/quant.go:236-248 */

/* ---- dot products / GEMV ------------------------------------------------- */
/* variant 0 = generic Go kernels (ml/matmul_q8.go:237-429,679-744),
 * variant 1 = AVX2 wrappers + asm (ml/matmul_q8_kernels_amd64.go:15-224,
 *             ml/dot_int8_f32_avx2_amd64.s:4-45). */
float or_dot(uint32_t type, const uint8_t *row, const float *x, int n, int variant);
/* out[m, r] = dot(W[r,:], a[m,:]) ; ml/matmul_q8.go:93-139 */
int or_gemv(uint32_t type, const uint8_t *w, int rows, int cols, const float *a, int m,
            float *out, int variant, int threads);

/* ---- elementwise / normalisation ---------------------------------------- */
void or_layernorm(float *dst, const float *src, const float *w, const float *b, int rows, int c,
                  float eps);                                       /* ml/ops.go:153-202 */
void or_gelu(float *x, int n);                                      /* ml/ops.go:102-122 */
float or_fast_exp(float x);                                         /* ml/attention.go:34-61 */
void or_softmax_fast(float *row, int n);                            /* ml/attention.go:93-131 */
void or_softmax_exact(float *row, int n);                           /* ml/attention.go:133-171 */
/* q [heads,Tq,hd], k/v [heads,Tk,hd] -> out [heads,Tq,hd]; ml/attention.go:193-281 */
void or_sdpa(const float *q, const float *k, const float *v, int heads, int tq, int tk, int hd,
             int causal, int fast_exp, float *out, float *weights);

/* ---- sampling ------------------------------------------------------------ */
/* model/decoder.go:1140-1167 (returns modified copy in out) */
void or_repetition_penalty(const float *logits, int n, const int32_t *hist, int hist_len,
                           float penalty, int window, float *out);
/* model/decoder.go:996-1059 without the top-p fallback */
int32_t or_sample_greedy(const float *logits, int n, float temperature, int suppress_nst,
                         float no_speech_thold, int32_t eot);
/* model/decoder.go:1068-1136 ; returns k entries sorted by logprob desc */
int or_topk(const float *logits, int n, int k, float temperature, int32_t *tok, float *logprob);

/* ---- decoder model --------------------------------------------------------- */
typedef struct {
    const char *name;      /* reference tensor name or HF alias (model/compat.go:31-148) */
    uint32_t type;         /* gguf QuantType: 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 6 Q5_0, 7 Q5_1, 8 Q8_0 */
    uint32_t ndim;
    uint64_t shape[4];     /* as stored in the GGUF descriptor (rows first) */
    const void *data;
    uint64_t nbytes;
} or_tensor;

typedef struct {
    /* whisper.decoder.* / whisper.vocab.size metadata, 0 = absent (decoder.go:101-105) */
    uint32_t n_head, n_layer, n_ctx, n_state, n_vocab;
} or_meta;

typedef struct {
    /* whisper.encoder.* / whisper.audio.mel_count metadata, 0 = absent (encoder.go:63-67) */
    uint32_t n_head, n_layer, n_ctx, n_state, n_mels;
} or_enc_meta;

typedef struct or_model or_model;
typedef struct or_state or_state;

or_model *or_model_create(const or_tensor *t, int n, const or_meta *meta, int dot_variant,
                          int threads);                             /* model/decoder.go:97-303 */
void or_model_destroy(or_model *m);
void or_model_hparams(const or_model *m, int32_t *out5);            /* vocab,state,head,layer,ctx */
void or_model_set_eot(or_model *m, int32_t eot);                    /* model/decoder.go:85-94 */
void or_model_set_fast_exp(or_model *m, int on);                    /* ml/attention.go:18-22 */
/* n > 1: the forward's batch-1 GEMVs split their rows over n threads; every
 * output element is the same dot as in the serial loop (fixture generation). */
void or_model_set_forward_threads(or_model *m, int n);

or_state *or_state_create(const or_model *m, const int32_t *prompt, int plen); /* decoder.go:306-365 */
void or_state_destroy(or_state *s);
void or_state_reset(const or_model *m, or_state *s, const int32_t *tokens, int n); /* decoder.go:367-386 */
int or_state_push(or_state *s, int32_t tok);
/* One forward for the last token of the state; logits [n_vocab]. decoder.go:745-833 */
int or_forward(const or_model *m, or_state *s, const float *enc, int enc_len, float *logits);
/* Precompute cross K/V for all layers with `threads` workers (decoder.go:923-940). */
int or_state_prepare_cross(const or_model *m, or_state *s, const float *enc, int enc_len);

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
} or_decode_params;

/* Whole Decode (decoder.go:401-726) without vocab-dependent retries. Writes the
 * full token sequence (prompt + generated) into out (capacity cap) and its
 * length into out_len. Returns 0 on success. */
int or_decode(const or_model *m, const float *enc, int enc_len, const or_decode_params *p,
              int32_t *out, int cap, int32_t *out_len);

/* Beam search with every beam exposed (test hook for the in-place reuse of
 * decoder.go:627-660): beam i's tokens at out + i*cap, lens[i], scores[i], in
 * the order of the final beams slice; *nbeams = its length. step_margin (may be
 * NULL) receives per step the smallest gap between different normalised scores
 * among the first beam_size + 1 sorted candidates (INFINITY if none). */
int or_beam_run(const or_model *m, const float *enc, int enc_len, const or_decode_params *p, int32_t *out, int cap,
                int32_t *lens, float *scores, int32_t *nbeams, float *step_margin, int margin_cap);

/* Go 1.25 sort.Slice (pdqsort_func) of n keys with less(i,j) = norm[i] > norm[j],
 * carrying id[] along (the restatement the beam prune uses, decoder.go:1462-1475). */
void or_go_sort_norm(float *norm, int32_t *id, int n);

const char *or_last_error(void);


/* ---- encoder (model/encoder.go) ----------------------------------------- */
typedef struct or_encoder or_encoder;
or_encoder *or_encoder_create(const or_tensor *t, int n, const or_enc_meta *meta, int dot_variant,
                              int threads);                         /* model/encoder.go:58-263 */
void or_encoder_destroy(or_encoder *e);
void or_encoder_hparams(const or_encoder *e, int32_t *out5);        /* mels,state,head,layer,ctx */
void or_encoder_set_fast_exp(or_encoder *e, int on);               /* ml/attention.go:18-22 */
/* Encode (encoder.go:265-338): mel [n_mels, T] -> out [T', d]; returns T' or -1. */
int or_encode(const or_encoder *e, const float *mel, int n_mels, int T, float *out);
/* ml/conv.go:19-70; returns T' */
int or_conv1d(const float *in, int in_c, int t, const float *w, const float *bias, int out_c, int kernel, int stride,
              float *out);

#ifdef __cplusplus
}
#endif
#endif
