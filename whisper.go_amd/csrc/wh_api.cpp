// C ABI of libwhisper_hip.so (declared in include/whisper_hip.h).
#include <hip/hip_runtime_api.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "wh_internal.h"

namespace wh {

static thread_local std::string g_error;
void set_error(const std::string &msg) { g_error = msg; }
int fail(int code, const std::string &msg) {
    g_error = msg;
    return code;
}

int model_create(const wh_tensor *tensors, int32_t n, const wh_meta *meta, int32_t device, wh_model **out);
void model_free(wh_model *m);
int encoder_create(const wh_tensor *tensors, int32_t n, const wh_enc_meta *meta, int32_t device, wh_encoder **out);
void encoder_free(wh_encoder *e);
int encoder_hparams(const wh_encoder *e, int32_t *o);
int encode(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out, int32_t out_cap,
           int32_t *out_rows, const volatile int32_t *cancel);
int encode_device(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out, int32_t out_cap,
                  int32_t *out_rows, const volatile int32_t *cancel);
int seq_create(const wh_model *m, int32_t S, const float *const *encs, int32_t enc_len, int32_t enc_dim, int32_t shared,
               wh_seq **out, int32_t dev);
int seq_set_tokens(wh_seq *s, int32_t i, const int32_t *tokens, int32_t n, int32_t reset_kv);
int seq_step_greedy(wh_seq *s, const int32_t *active, float temperature, int32_t suppress_nst, float nst,
                    int32_t *out_ids, float *out_logits);
int seq_step_topk(wh_seq *s, const int32_t *active, int32_t k, float temperature, int32_t *out_tok, float *out_lp,
                  float *out_logits);
void seq_destroy(wh_seq *s);
int seq_set_profiling(wh_seq *s, int32_t enable);
int seq_generate(wh_seq *s, int32_t n, float temperature, int32_t suppress_nst, float nst, int32_t max_len,
                 int32_t *out_ids, int32_t *out_n);
int seq_profile_count(wh_seq *s, int32_t *n);
int seq_persistent(wh_seq *s, int32_t *out, int64_t *launches);
int seq_profile_get(wh_seq *s, int32_t i, char *name, int32_t cap, double *ms, int64_t *launches, double *bytes);
int decode_greedy_batch(const wh_model *m, int32_t S, const float *const *encs, int32_t enc_len, int32_t enc_dim,
                        const wh_decode_params *params, int32_t *out_tokens, int32_t cap, int32_t *out_lens,
                        const volatile int32_t *cancel, int32_t dev);
int32_t last_decode_steps();
int decode_beam(const wh_model *m, const float *enc, int32_t enc_len, int32_t enc_dim, const wh_decode_params *p,
                int32_t *out_tokens, int32_t cap, int32_t *out_len, const volatile int32_t *cancel, int32_t dev);

// ---- GGUF v2/v3 reader (internal/gguf/gguf.go:52-135, metadata.go, tensor.go) ----
namespace {

struct Reader {
    const uint8_t *p, *end;
    bool ok = true;
    template <typename T>
    T get() {
        T v{};
        if ((size_t)(end - p) < sizeof(T)) { ok = false; return v; }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t)(end - p) < n) { ok = false; return ""; }
        std::string s((const char *)p, (size_t)n);
        p += n;
        return s;
    }
    // skip one metadata value of type t (metadata.go:42-145)
    void skip(uint32_t t, std::map<std::string, uint32_t> *u32, const std::string &key) {
        switch (t) {
        case 0: case 1: case 7: get<uint8_t>(); break;
        case 2: case 3: get<uint16_t>(); break;
        case 4: { uint32_t v = get<uint32_t>(); if (u32) (*u32)[key] = v; break; }
        case 5: case 6: get<uint32_t>(); break;
        case 8: str(); break;
        case 9: {
            uint32_t et = get<uint32_t>();
            uint64_t cnt = get<uint64_t>();
            for (uint64_t i = 0; i < cnt && ok; i++) skip(et, nullptr, key);
            break;
        }
        case 10: case 11: case 12: get<uint64_t>(); break;
        default: ok = false; break;
        }
    }
};

}  // namespace

// A GGUF v2/v3 file mapped read-only (gguf.go:52-135): the tensor table points
// into the mapping, the u32 metadata values are kept by key.
struct GgufMap {
    void *mp = nullptr;
    size_t size = 0;
    std::vector<std::string> names;
    std::vector<wh_tensor> table;
    std::map<std::string, uint32_t> u32;
    uint32_t get(const char *k) const {
        auto it = u32.find(k);
        return it == u32.end() ? 0u : it->second;
    }
    ~GgufMap() {
        if (mp) munmap(mp, size);
    }
};

int gguf_map(const char *path, GgufMap &g) {
    if (!path) return fail(WH_ERR_INVALID, "gguf: open: null argument");
    int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(WH_ERR_INVALID, std::string("gguf: open: ") + path + ": " + std::strerror(errno));
    struct stat stt;
    if (fstat(fd, &stt) != 0 || stt.st_size < 24) { close(fd); return fail(WH_ERR_INVALID, "gguf: read magic: short file"); }
    const size_t size = (size_t)stt.st_size;
    void *mp = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (mp == MAP_FAILED) return fail(WH_ERR_INVALID, "gguf: mmap failed");
    g.mp = mp;
    g.size = size;
    Reader r{(const uint8_t *)mp, (const uint8_t *)mp + size};
    if (std::memcmp(r.p, "GGUF", 4) != 0) return fail(WH_ERR_INVALID, "gguf: invalid magic");
    r.p += 4;
    uint32_t version = r.get<uint32_t>();
    if (version != 2 && version != 3) return fail(WH_ERR_UNSUPPORTED, "gguf: unsupported version: " + std::to_string(version));
    uint64_t nt = r.get<uint64_t>(), nm = r.get<uint64_t>();
    for (uint64_t i = 0; i < nm && r.ok; i++) {
        std::string key = r.str();
        uint32_t t = r.get<uint32_t>();
        r.skip(t, &g.u32, key);
    }
    if (!r.ok) return fail(WH_ERR_INVALID, "gguf: metadata: truncated");
    struct Desc { std::vector<uint64_t> shape; uint32_t type; uint64_t off; };
    std::vector<Desc> descs(nt);
    g.names.resize(nt);
    for (uint64_t i = 0; i < nt && r.ok; i++) {
        g.names[i] = r.str();
        uint32_t nd = r.get<uint32_t>();
        if (nd > 4) return fail(WH_ERR_INVALID, "gguf: tensor: too many dimensions");
        for (uint32_t j = 0; j < nd; j++) descs[i].shape.push_back(r.get<uint64_t>());
        descs[i].type = r.get<uint32_t>();
        descs[i].off = r.get<uint64_t>();
    }
    if (!r.ok) return fail(WH_ERR_INVALID, "gguf: tensor info: truncated");
    uint64_t align = 32;
    auto ai = g.u32.find("general.alignment");
    if (ai != g.u32.end() && ai->second > 0) align = ai->second;
    const uint64_t pos = (uint64_t)(r.p - (const uint8_t *)mp);
    const uint64_t data_start = (pos + align - 1) / align * align;
    g.table.resize(nt);
    for (uint64_t i = 0; i < nt; i++) {
        wh_tensor &t = g.table[i];
        const Desc &d = descs[i];
        t.name = g.names[i].c_str();
        t.type = d.type;
        t.ndim = (uint32_t)d.shape.size();
        uint64_t n = 1;
        for (uint32_t j = 0; j < t.ndim; j++) { t.shape[j] = d.shape[j]; n *= d.shape[j]; }
        const uint64_t bytes = gguf_row_bytes(d.type, n);
        t.data = (const uint8_t *)mp + data_start + d.off;
        t.nbytes = (data_start + d.off <= size) ? std::min<uint64_t>(bytes, size - data_start - d.off) : 0;
    }
    return WH_OK;
}

int model_load_gguf(const char *path, int32_t device, wh_model **out) {
    if (!path || !out) return fail(WH_ERR_INVALID, "gguf: open: null argument");
    *out = nullptr;
    GgufMap g;
    int rc = gguf_map(path, g);
    if (rc) return rc;
    wh_meta meta{};
    meta.n_head = g.get("whisper.decoder.attention.head_count");
    meta.n_layer = g.get("whisper.decoder.layer_count");
    meta.n_ctx = g.get("whisper.decoder.context_length");
    meta.n_state = g.get("whisper.decoder.embedding_length");
    meta.n_vocab = g.get("whisper.vocab.size");
    if (!meta.n_vocab) meta.n_vocab = g.get("whisper.n_vocab");
    return model_create(g.table.data(), (int32_t)g.table.size(), &meta, device, out);
}

// NewEncoder over a GGUF file (encoder.go:58-67: whisper.encoder.* metadata,
// the mel band count under either key).
int encoder_load_gguf(const char *path, int32_t device, wh_encoder **out) {
    if (!path || !out) return fail(WH_ERR_INVALID, "gguf: open: null argument");
    *out = nullptr;
    GgufMap g;
    int rc = gguf_map(path, g);
    if (rc) return rc;
    wh_enc_meta meta{};
    meta.n_head = g.get("whisper.encoder.attention.head_count");
    meta.n_layer = g.get("whisper.encoder.layer_count");
    meta.n_ctx = g.get("whisper.encoder.context_length");
    meta.n_state = g.get("whisper.encoder.embedding_length");
    meta.n_mels = g.get("whisper.audio.mel_count");
    if (!meta.n_mels) meta.n_mels = g.get("whisper.n_mels");
    return encoder_create(g.table.data(), (int32_t)g.table.size(), &meta, device, out);
}

}  // namespace wh

using namespace wh;

extern "C" {

const char *wh_last_error(void) { return g_error.c_str(); }
const char *wh_version(void) { return "whisper-hip 0.1 (gfx950)"; }

int wh_device_count(int32_t *count) {
    if (!count) return fail(WH_ERR_INVALID, "null argument");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    return WH_OK;
}

int wh_dev_malloc(uint64_t bytes, int32_t device, void **out) {
    if (!out) return fail(WH_ERR_INVALID, "null argument");
    *out = nullptr;
    WH_HIP(hipSetDevice(device));
    WH_HIP(hipMalloc(out, bytes ? bytes : 1));
    return WH_OK;
}
int wh_dev_free(void *p) {
    if (p) WH_HIP(hipFree(p));
    return WH_OK;
}
int wh_memcpy(void *dst, const void *src, uint64_t bytes, int32_t kind) {
    if (!bytes) return WH_OK;
    if (!dst || !src) return fail(WH_ERR_INVALID, "memcpy: null pointer");
    hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    if (kind < 0 || kind > 2) return fail(WH_ERR_INVALID, "memcpy: kind must be 0, 1 or 2");
    WH_HIP(hipMemcpy(dst, src, bytes, k));
    return WH_OK;
}
int wh_stream_create(int32_t device, void **out) {
    if (!out) return fail(WH_ERR_INVALID, "null argument");
    WH_HIP(hipSetDevice(device));
    hipStream_t s;
    WH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *out = (void *)s;
    return WH_OK;
}
int wh_stream_destroy(void *s) {
    if (s) WH_HIP(hipStreamDestroy((hipStream_t)s));
    return WH_OK;
}
int wh_stream_sync(void *s) {
    WH_HIP(hipStreamSynchronize((hipStream_t)s));
    return WH_OK;
}
int wh_event_create(void **out) {
    if (!out) return fail(WH_ERR_INVALID, "null argument");
    hipEvent_t e;
    WH_HIP(hipEventCreate(&e));
    *out = (void *)e;
    return WH_OK;
}
int wh_event_destroy(void *e) {
    if (e) WH_HIP(hipEventDestroy((hipEvent_t)e));
    return WH_OK;
}
int wh_event_record(void *e, void *s) {
    WH_HIP(hipEventRecord((hipEvent_t)e, (hipStream_t)s));
    return WH_OK;
}
int wh_event_elapsed(void *a, void *b, float *ms) {
    if (!ms) return fail(WH_ERR_INVALID, "null argument");
    WH_HIP(hipEventSynchronize((hipEvent_t)b));
    WH_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return WH_OK;
}

uint64_t wh_row_bytes(uint32_t type, uint64_t n) { return gguf_row_bytes(type, n); }

int wh_quantize(uint32_t type, const float *src, uint64_t n, void *dst, uint64_t dst_bytes, int32_t threads) {
    if ((!src || !dst) && n) return fail(WH_ERR_INVALID, "gguf: quantize: null buffer");
    return quantize(type, src, n, (uint8_t *)dst, dst_bytes, threads);
}

int wh_should_quantize(const char *name) { return should_quantize(name); }
uint16_t wh_f32_to_f16(float f) { return f32_to_f16(f); }
float wh_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

int wh_dequantize(uint32_t type, const void *raw, uint64_t nbytes, uint64_t n, float *out, int32_t device) {
    if (!out || (!raw && n)) return fail(WH_ERR_INVALID, "dequantize: null buffer");
    if (n == 0) return WH_OK;
    if (n > (uint64_t)1 << 31) return fail(WH_ERR_INVALID, "dequantize: too many elements");
    // one row of n elements, decoded by the kernels' device routine
    DevMat m;
    int rc = devmat_plan(m, type, 1, (int32_t)n);
    if (rc) return rc;
    WH_HIP(hipSetDevice(device));
    if ((rc = devmat_upload_typed(m, type, (const uint8_t *)raw, nbytes))) return rc;
    float *d = nullptr;
    hipError_t e = hipMalloc(&d, n * sizeof(float));
    if (e == hipSuccess) {
        rc = launch_dequant_rows(m, 0, 1, d, nullptr);
        if (!rc) {
            e = hipMemcpy(out, d, n * sizeof(float), hipMemcpyDeviceToHost);
            if (e != hipSuccess) rc = fail(WH_ERR_HIP, std::string("hip: dequantize copy: ") + hipGetErrorString(e));
        }
        (void)hipFree(d);
    } else {
        rc = fail(WH_ERR_NOMEM, "hip: dequantize alloc failed");
    }
    devmat_free(m);
    return rc;
}

int wh_dequantize_noalloc(uint32_t type, const void *raw, uint64_t nbytes, uint64_t n, float *out, int32_t device) {
    return dequantize_noalloc(type, raw, nbytes, n, out, device);
}

int wh_matrix_create(uint32_t type, int32_t rows, int32_t cols, const void *raw, uint64_t nbytes, int32_t device,
                     wh_matrix **out) {
    if (!out || !raw) return fail(WH_ERR_INVALID, "NewQuantizedMatrix: null argument");
    *out = nullptr;
    wh_matrix *w = new wh_matrix();
    w->device = device;
    int rc = devmat_plan(w->m, type, rows, cols);
    const uint64_t need = (uint64_t)rows * gguf_row_bytes(type, (uint64_t)cols);
    if (!rc && nbytes < need)
        rc = fail(WH_ERR_INVALID,
                  "NewQuantizedMatrix: short data got=" + std::to_string(nbytes) + " need=" + std::to_string(need));
    if (!rc) {
        hipError_t e = hipSetDevice(device);
        rc = e == hipSuccess ? devmat_upload_typed(w->m, type, (const uint8_t *)raw, nbytes)
                             : fail(WH_ERR_HIP, "hip: set device failed");
    }
    if (rc) { delete w; return rc; }
    *out = w;
    return WH_OK;
}

int wh_matrix_destroy(wh_matrix *m) {
    if (!m) return WH_OK;
    devmat_free(m->m);
    delete m;
    return WH_OK;
}

int wh_matrix_bytes(const wh_matrix *m, uint64_t *bytes) {
    if (!m || !bytes) return fail(WH_ERR_INVALID, "null argument");
    *bytes = m->m.algo_bytes;
    return WH_OK;
}

int wh_gemv(const wh_matrix *w, const float *x, int32_t batch, float *y, void *stream) {
    if (!w || !x || !y) return fail(WH_ERR_INVALID, "MatMulQuantTransBInto: null argument");
    const DevMat *mp = &w->m;
    GemvIn in{x, w->m.cols};
    GemvOut o;
    o.y = y;
    o.ldy = w->m.rows;
    return launch_gemv(&mp, &in, &o, 1, batch, (hipStream_t)stream);
}

int wh_model_create(const wh_tensor *tensors, int32_t n, const wh_meta *meta, int32_t device, wh_model **out) {
    return model_create(tensors, n, meta, device, out);
}
int wh_model_load_gguf(const char *path, int32_t device, wh_model **out) { return model_load_gguf(path, device, out); }
int wh_encoder_create(const wh_tensor *tensors, int32_t n, const wh_enc_meta *meta, int32_t device,
                      wh_encoder **out) {
    return encoder_create(tensors, n, meta, device, out);
}
int wh_encoder_load_gguf(const char *path, int32_t device, wh_encoder **out) {
    return encoder_load_gguf(path, device, out);
}
int wh_encoder_destroy(wh_encoder *e) {
    encoder_free(e);
    return WH_OK;
}
int wh_encoder_hparams(const wh_encoder *e, int32_t *out5) { return encoder_hparams(e, out5); }
int wh_encode(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out, int32_t out_cap,
              int32_t *out_rows, const volatile int32_t *cancel) {
    return encode(e, mel, n_mels, T, out, out_cap, out_rows, cancel);
}
int wh_encode_device(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out, int32_t out_cap,
                     int32_t *out_rows, const volatile int32_t *cancel) {
    return encode_device(e, mel, n_mels, T, out, out_cap, out_rows, cancel);
}
int wh_model_destroy(wh_model *m) {
    model_free(m);
    return WH_OK;
}
int wh_model_hparams(const wh_model *m, int32_t *o) {
    if (!m || !o) return fail(WH_ERR_INVALID, "null argument");
    o[0] = m->n_vocab; o[1] = m->n_state; o[2] = m->n_head; o[3] = m->n_layer; o[4] = m->n_ctx;
    return WH_OK;
}
int wh_model_set_eot(wh_model *m, int32_t eot) {
    if (!m) return fail(WH_ERR_INVALID, "null argument");
    m->eot = eot;
    return WH_OK;
}
int wh_model_weight_bytes(const wh_model *m, uint64_t *bytes) {
    if (!m || !bytes) return fail(WH_ERR_INVALID, "null argument");
    *bytes = m->weight_bytes;
    return WH_OK;
}
int wh_model_set_attention_mode(wh_model *m, int32_t mode) {
    if (!m || (mode != 0 && mode != 1)) return fail(WH_ERR_INVALID, "attention mode must be 0 or 1");
    m->attn_mode = mode;
    return WH_OK;
}

int wh_last_decode_steps(int32_t *out) {
    if (!out) return fail(WH_ERR_INVALID, "null argument");
    *out = last_decode_steps();
    return WH_OK;
}

int wh_decode(const wh_model *m, const float *enc, int32_t enc_len, int32_t enc_dim, const wh_decode_params *p,
              int32_t *out_tokens, int32_t cap, int32_t *out_len, const volatile int32_t *cancel) {
    if (!m || !enc || !p || !out_tokens || !out_len) return fail(WH_ERR_INVALID, "model: decode: null argument");
    *out_len = 0;
    if (p->beam_size > 1) return decode_beam(m, enc, enc_len, enc_dim, p, out_tokens, cap, out_len, cancel, 0);
    return decode_greedy_batch(m, 1, &enc, enc_len, enc_dim, p, out_tokens, cap, out_len, cancel, 0);
}

int wh_decode_device(const wh_model *m, const float *enc, int32_t enc_len, int32_t enc_dim, const wh_decode_params *p,
                     int32_t *out_tokens, int32_t cap, int32_t *out_len, const volatile int32_t *cancel) {
    if (!m || !enc || !p || !out_tokens || !out_len) return fail(WH_ERR_INVALID, "model: decode: null argument");
    *out_len = 0;
    if (p->beam_size > 1) return decode_beam(m, enc, enc_len, enc_dim, p, out_tokens, cap, out_len, cancel, 1);
    return decode_greedy_batch(m, 1, &enc, enc_len, enc_dim, p, out_tokens, cap, out_len, cancel, 1);
}

int wh_decode_batch(const wh_model *m, int32_t n, const float *const *encs, int32_t enc_len, int32_t enc_dim,
                    const wh_decode_params *params, int32_t *out_tokens, int32_t cap, int32_t *out_lens,
                    const volatile int32_t *cancel) {
    if (!m || !encs || !params || !out_tokens || !out_lens) return fail(WH_ERR_INVALID, "model: decode: null argument");
    return decode_greedy_batch(m, n, encs, enc_len, enc_dim, params, out_tokens, cap, out_lens, cancel, 0);
}

int wh_seq_create(const wh_model *m, int32_t n, const float *const *encs, int32_t enc_len, int32_t enc_dim,
                  int32_t shared, wh_seq **out) {
    return seq_create(m, n, encs, enc_len, enc_dim, shared, out, 0);
}
int wh_seq_create_device(const wh_model *m, int32_t n, const float *const *encs, int32_t enc_len, int32_t enc_dim,
                         int32_t shared, wh_seq **out) {
    return seq_create(m, n, encs, enc_len, enc_dim, shared, out, 1);
}
int wh_seq_destroy(wh_seq *s) {
    seq_destroy(s);
    return WH_OK;
}
int wh_seq_set_tokens(wh_seq *s, int32_t stream, const int32_t *tokens, int32_t n, int32_t reset_kv) {
    return seq_set_tokens(s, stream, tokens, n, reset_kv);
}
int wh_seq_step_greedy(wh_seq *s, const int32_t *active, float temperature, int32_t suppress_nst, float nst,
                       int32_t *out_ids, float *out_logits) {
    return seq_step_greedy(s, active, temperature, suppress_nst, nst, out_ids, out_logits);
}
int wh_seq_step_topk(wh_seq *s, const int32_t *active, int32_t k, float temperature, int32_t *out_tok,
                     float *out_logprob, float *out_logits) {
    if (!out_tok || !out_logprob) return fail(WH_ERR_INVALID, "seq: null output");
    return seq_step_topk(s, active, k, temperature, out_tok, out_logprob, out_logits);
}
int wh_seq_generate(wh_seq *s, int32_t n, float temperature, int32_t suppress_nst, float nst, int32_t max_len,
                    int32_t *out_ids, int32_t *out_n) {
    return seq_generate(s, n, temperature, suppress_nst, nst, max_len, out_ids, out_n);
}
int wh_seq_persistent(wh_seq *s, int32_t *out, int64_t *launches) { return seq_persistent(s, out, launches); }
int wh_seq_set_profiling(wh_seq *s, int32_t enable) { return seq_set_profiling(s, enable); }
int wh_seq_profile_count(wh_seq *s, int32_t *n) { return seq_profile_count(s, n); }
int wh_seq_profile_get(wh_seq *s, int32_t i, char *name, int32_t cap, double *ms, int64_t *launches, double *bytes) {
    return seq_profile_get(s, i, name, cap, ms, launches, bytes);
}

}  // extern "C"
