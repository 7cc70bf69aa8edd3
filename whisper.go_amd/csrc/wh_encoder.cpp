// Encoder model creation and forward (internal/model/encoder.go:58-396) on the
// device: weights uploaded once (quantised matrices stay quantised), the conv
// stem and every projection as fp32 matrix-core products (k_cross_gemm), the
// attention of each head over all frames in one kernel (wh_encoder.hip).
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "wh_internal.h"
#include "wh_load.h"

struct wh_encoder {
    int32_t device = 0;
    int32_t n_mels = 0, n_state = 0, n_head = 0, n_layer = 0, n_ctx = 0;
    int32_t k1 = 0;                        // conv1 product width: 3 n_mels padded to 32
    wh::DevMat conv1, conv2;               // [d, k1] and [d, 3d] f32 (conv weights flattened)
    float *conv1b = nullptr, *conv2b = nullptr, *pos = nullptr, *lnw = nullptr, *lnb = nullptr;
    struct Block {
        float *ln1w, *ln1b, *qb, *vb, *ob, *ln2w, *ln2b, *fc1b, *fc2b;
        wh::DevMat q, k, v, o, fc1, fc2;
    };
    std::vector<Block> blocks;
    void *vec_alloc = nullptr;
    // the forward's stream and workspace (sized for T = 2 n_ctx on first use),
    // held for the encoder's lifetime; one encode at a time per handle
    mutable hipStream_t st = nullptr;
    mutable float *ws = nullptr;
    mutable std::mutex mu;
};

namespace wh {

void encoder_free(wh_encoder *e) {
    if (!e) return;
    devmat_free(e->conv1);
    devmat_free(e->conv2);
    for (auto &b : e->blocks) {
        DevMat *ms[] = {&b.q, &b.k, &b.v, &b.o, &b.fc1, &b.fc2};
        for (DevMat *m : ms) devmat_free(*m);
    }
    if (e->vec_alloc) (void)hipFree(e->vec_alloc);
    if (e->ws) (void)hipFree(e->ws);
    if (e->st) (void)hipStreamDestroy(e->st);
    delete e;
}

namespace {

// ml.Transpose of a [n0, n1, n2] tensor by the axis permutation (i0, i1, i2).
std::vector<float> transpose3(const std::vector<float> &src, const uint64_t *sh, int i0, int i1, int i2) {
    const uint64_t n[3] = {sh[0], sh[1], sh[2]};
    std::vector<float> o(src.size());
    for (uint64_t a = 0; a < n[0]; a++)
        for (uint64_t b = 0; b < n[1]; b++)
            for (uint64_t c = 0; c < n[2]; c++) {
                const uint64_t idx[3] = {a, b, c};
                o[(idx[i0] * n[i1] + idx[i1]) * n[i2] + idx[i2]] = src[(a * n[1] + b) * n[2] + c];
            }
    return o;
}

// A [rows, cols] float matrix padded with zero columns to width, uploaded as f32.
int upload_padded(const std::vector<float> &f, int rows, int cols, int width, DevMat &m) {
    std::vector<float> p((size_t)rows * width, 0.0f);
    for (int r = 0; r < rows; r++) std::memcpy(&p[(size_t)r * width], &f[(size_t)r * cols], sizeof(float) * cols);
    int rc = devmat_plan(m, WH_TYPE_F32, rows, width);
    if (rc) return rc;
    return devmat_upload_typed(m, WH_TYPE_F32, (const uint8_t *)p.data(), p.size() * 4);
}

}  // namespace

int encoder_create(const wh_tensor *tensors, int32_t n, const wh_enc_meta *meta, int32_t device, wh_encoder **out) {
    if (!out) return fail(WH_ERR_INVALID, "model: encoder: null output handle");
    *out = nullptr;
    if (n < 0 || (n > 0 && !tensors)) return fail(WH_ERR_INVALID, "model: encoder: invalid tensor table");
    Table tab;
    for (int32_t i = 0; i < n; i++) {
        if (!tensors[i].name) return fail(WH_ERR_INVALID, "model: encoder: tensor without a name");
        if (tensors[i].ndim > 4) return fail(WH_ERR_INVALID, std::string("model: encoder: too many dims for ") + tensors[i].name);
        tab.byname[tensors[i].name] = &tensors[i];
    }
    uint32_t n_head = meta ? meta->n_head : 0, n_layer = meta ? meta->n_layer : 0, n_ctx = meta ? meta->n_ctx : 0;
    uint32_t n_state = meta ? meta->n_state : 0, n_mels = meta ? meta->n_mels : 0;
    // encoder.go:69-119
    if (n_layer == 0)
        while (tab.resolve("encoder.blocks." + std::to_string(n_layer) + ".attn.query.weight")) n_layer++;
    if (n_state == 0) {
        const wh_tensor *b = tab.resolve("encoder.conv1.bias");
        if (!b) return not_found("encoder.conv1.bias");
        if (b->ndim != 1 || b->shape[0] == 0) return fail(WH_ERR_INVALID, "model: encoder: invalid conv1.bias shape");
        n_state = (uint32_t)b->shape[0];
    }
    if (const wh_tensor *aq = tab.resolve("encoder.blocks.0.attn.query.weight"))
        if (aq->ndim == 2 && aq->shape[0] == aq->shape[1] && aq->shape[0] > 0) n_state = (uint32_t)aq->shape[0];
    const wh_tensor *pe = tab.resolve("encoder.positional_embedding");
    if (n_ctx == 0) {
        if (!pe) return not_found("encoder.positional_embedding");
        if (pe->ndim != 2) return fail(WH_ERR_INVALID, "model: encoder: invalid positional embedding shape");
        n_ctx = (pe->shape[0] == n_state && pe->shape[1] != n_state) ? (uint32_t)pe->shape[1] : (uint32_t)pe->shape[0];
    }
    if (n_head == 0) {
        if (n_state % 64 != 0)
            return fail(WH_ERR_INVALID,
                        "model: encoder: cannot infer head count from embedding length " + std::to_string(n_state));
        n_head = n_state / 64;
    }
    if (n_state % n_head != 0 || n_state % 4 != 0)
        return fail(WH_ERR_INVALID, "model: encoder: inconsistent hyper-parameters");
    WH_HIP(hipSetDevice(device));
    std::unique_ptr<wh_encoder, void (*)(wh_encoder *)> e(new wh_encoder(), encoder_free);
    e->device = device;
    e->n_state = (int32_t)n_state;
    e->n_head = (int32_t)n_head;
    e->n_layer = (int32_t)n_layer;
    e->n_ctx = (int32_t)n_ctx;
    const int d = e->n_state;
    int rc;
    // conv1 (encoder.go:121-150): [d, n_mels, 3], the legacy [n_mels, d, 3], or [3, n_mels, d]
    {
        const wh_tensor *t = tab.resolve("encoder.conv1.weight");
        if (!t) return not_found("encoder.conv1.weight");
        if (t->ndim != 3) return fail(WH_ERR_INVALID, "model: encoder: invalid conv1.weight shape");
        std::vector<float> f;
        if ((rc = load_f32(t, f))) return rc;
        if ((int64_t)t->shape[0] == d && t->shape[1] > 0 && t->shape[2] == 3) {
            if (!n_mels) n_mels = (uint32_t)t->shape[1];
        } else if ((int64_t)t->shape[1] == d && t->shape[0] > 0 && t->shape[2] == 3) {
            f = transpose3(f, t->shape, 1, 0, 2);
            if (!n_mels) n_mels = (uint32_t)t->shape[0];
        } else if (t->shape[0] == 3 && (int64_t)t->shape[2] == d && t->shape[1] > 0) {
            f = transpose3(f, t->shape, 2, 1, 0);
            if (!n_mels) n_mels = (uint32_t)t->shape[1];
        } else {
            return fail(WH_ERR_INVALID, "model: encoder: unsupported conv1.weight shape");
        }
        if ((uint64_t)n_mels * 3 * d != f.size())
            return fail(WH_ERR_INVALID, "model: encoder: conv1.weight does not match n_mels");
        e->n_mels = (int32_t)n_mels;
        e->k1 = (3 * e->n_mels + 31) / 32 * 32;
        if ((rc = upload_padded(f, d, 3 * e->n_mels, e->k1, e->conv1))) return rc;
    }
    // conv2 (encoder.go:156-170): [d, d, 3], [3, d, d], else the (1, 0, 2) transpose
    {
        const wh_tensor *t = tab.resolve("encoder.conv2.weight");
        if (!t) return not_found("encoder.conv2.weight");
        if (t->ndim != 3) return fail(WH_ERR_INVALID, "model: encoder: invalid conv2.weight shape");
        std::vector<float> f;
        if ((rc = load_f32(t, f))) return rc;
        if (f.size() != (size_t)3 * d * d) return fail(WH_ERR_INVALID, "model: encoder: invalid conv2.weight shape");
        if ((int64_t)t->shape[0] == d && (int64_t)t->shape[1] == d && t->shape[2] == 3) {
        } else if (t->shape[0] == 3 && (int64_t)t->shape[1] == d && (int64_t)t->shape[2] == d) {
            f = transpose3(f, t->shape, 2, 1, 0);
        } else {
            f = transpose3(f, t->shape, 1, 0, 2);
        }
        if ((rc = upload_padded(f, d, 3 * d, 3 * d, e->conv2))) return rc;
    }
    VecArena arena;
    if ((rc = load_vector(tab, "encoder.conv1.bias", arena, &e->conv1b, (size_t)d))) return rc;
    if ((rc = load_vector(tab, "encoder.conv2.bias", arena, &e->conv2b, (size_t)d))) return rc;
    {
        if (!pe) return not_found("encoder.positional_embedding");
        if (pe->ndim != 2) return fail(WH_ERR_INVALID, "model: encoder: invalid positional embedding shape");
        std::vector<float> f;
        if ((rc = load_f32(pe, f))) return rc;
        if ((int64_t)pe->shape[0] == d && (int64_t)pe->shape[1] == e->n_ctx) {
            std::vector<float> tr(f.size());
            for (int i = 0; i < d; i++)
                for (int j = 0; j < e->n_ctx; j++) tr[(size_t)j * d + i] = f[(size_t)i * e->n_ctx + j];
            f.swap(tr);
        }
        if (f.size() < (size_t)e->n_ctx * d) return fail(WH_ERR_INVALID, "model: encoder: positional embedding too small");
        arena.add(f, &e->pos);
    }
    e->blocks.resize(n_layer);
    for (uint32_t i = 0; i < n_layer; i++) {
        wh_encoder::Block &b = e->blocks[i];
        const std::string p = "encoder.blocks." + std::to_string(i) + ".";
        struct V { const char *suf; float **slot; size_t len; } vecs[] = {
            {"attn_ln.weight", &b.ln1w, (size_t)d}, {"attn_ln.bias", &b.ln1b, (size_t)d},
            {"attn.query.bias", &b.qb, (size_t)d},  {"attn.value.bias", &b.vb, (size_t)d},
            {"attn.out.bias", &b.ob, (size_t)d},    {"mlp_ln.weight", &b.ln2w, (size_t)d},
            {"mlp_ln.bias", &b.ln2b, (size_t)d},    {"mlp.0.bias", &b.fc1b, 4 * (size_t)d},
            {"mlp.2.bias", &b.fc2b, (size_t)d}};
        for (auto &v : vecs)
            if ((rc = load_vector(tab, p + v.suf, arena, v.slot, v.len))) return rc;
        struct M { const char *suf; DevMat *mat; int rows, cols; } mats[] = {
            {"attn.query.weight", &b.q, d, d}, {"attn.key.weight", &b.k, d, d},
            {"attn.value.weight", &b.v, d, d}, {"attn.out.weight", &b.o, d, d},
            {"mlp.0.weight", &b.fc1, 4 * d, d}, {"mlp.2.weight", &b.fc2, d, 4 * d}};
        for (auto &mm : mats)
            if ((rc = load_matrix(tab, p + mm.suf, mm.rows, mm.cols, *mm.mat))) return rc;
    }
    if ((rc = load_vector(tab, "encoder.ln_post.weight", arena, &e->lnw, (size_t)d))) return rc;
    if ((rc = load_vector(tab, "encoder.ln_post.bias", arena, &e->lnb, (size_t)d))) return rc;
    WH_HIP(hipMalloc(&e->vec_alloc, arena.host.size() * sizeof(float) + 256));
    WH_HIP(hipMemcpy(e->vec_alloc, arena.host.data(), arena.host.size() * sizeof(float), hipMemcpyHostToDevice));
    for (auto &f : arena.fix) *f.first = (float *)e->vec_alloc + f.second;
    // the forward's stream and code objects now, not in the first encode (the
    // runtime sets up a stream's hardware queue and loads code on first use)
    WH_HIP(hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking));
    if ((rc = warm_encoder_kernels()) || (rc = warm_kernels())) return rc;
    *out = e.release();
    return WH_OK;
}

int encoder_hparams(const wh_encoder *e, int32_t *o) {
    if (!e || !o) return fail(WH_ERR_INVALID, "model: encoder: null argument");
    o[0] = e->n_mels; o[1] = e->n_state; o[2] = e->n_head; o[3] = e->n_layer; o[4] = e->n_ctx;
    return WH_OK;
}

namespace {

// Frame-count rules of Encode (encoder.go:271-282): T = 2 n_ctx + 1 keeps the
// first n_mels * 2 n_ctx values of the buffer (the same base, row stride 2 n_ctx);
// T > 2 n_ctx is an error. Returns the frames the conv stem reads.
int frames(const wh_encoder *e, int32_t n_mels, int32_t T, int32_t out_cap, int *tout) {
    if (n_mels != e->n_mels || T <= 0)
        return fail(WH_ERR_INVALID, "model: encoder: mel must be [" + std::to_string(e->n_mels) + ", T], got [" +
                                      std::to_string(n_mels) + " " + std::to_string(T) + "]");
    if (T == 2 * e->n_ctx + 1) T = 2 * e->n_ctx;
    if (T > 2 * e->n_ctx)
        return fail(WH_ERR_INVALID, "model: encoder: T=" + std::to_string(T) + " > 2*n_audio_ctx=" +
                                        std::to_string(2 * e->n_ctx));
    if (out_cap < (T - 1) / 2 + 1) return fail(WH_ERR_INVALID, "model: encoder: output capacity too small");
    *tout = T;
    return WH_OK;
}

// Workspace of one forward at the largest frame count: mel staging, conv1
// staging and output, conv2 staging, x, ln, q, k, v, attn, h.
struct Work {
    float *dmel, *e1, *c1, *e2, *x, *xln, *q, *k, *v, *att, *h;
};
size_t carve(const wh_encoder *e, float *base, Work *w) {
    const int T = 2 * e->n_ctx, tp = e->n_ctx, d = e->n_state;
    size_t off = 0;
    auto take = [&](size_t n) { float *p = base ? base + off : nullptr; off += (n + 63) / 64 * 64; return p; };
    w->dmel = take((size_t)e->n_mels * T);
    w->e1 = take((size_t)T * e->k1);
    w->c1 = take((size_t)T * d);
    w->e2 = take((size_t)tp * 3 * d);
    float **xs[] = {&w->x, &w->xln, &w->q, &w->k, &w->v, &w->att};
    for (float **p : xs) *p = take((size_t)tp * d);
    w->h = take((size_t)tp * 4 * d);
    return off;
}

// The forward (encoder.go:284-338) of mel (device, [n_mels, T] rows T apart) into
// out (device, [T', d]) on the encoder's stream; returns once out is written.
int forward(const wh_encoder *e, const Work &w, const float *mel, int T, float *out, const volatile int32_t *cancel) {
    const int d = e->n_state, H = e->n_head, tp = (T - 1) / 2 + 1;
    const hipStream_t st = e->st;
    int rc;
    // conv stem (encoder.go:284-303): conv1 (stride 1) + GELU, conv2 (stride 2) + GELU,
    // frames first, plus the positional embedding of the first T' rows
    if ((rc = launch_im2col(mel, T, 1, e->n_mels, T, 1, T, e->k1, w.e1, st))) return rc;
    if ((rc = launch_cross_gemm(e->conv1, w.e1, T, e->conv1b, w.c1, st))) return rc;
    if ((rc = launch_gelu_add(w.c1, nullptr, (int64_t)T * d, st))) return rc;
    if ((rc = launch_im2col(w.c1, 1, d, d, T, 2, tp, 3 * d, w.e2, st))) return rc;
    if ((rc = launch_cross_gemm(e->conv2, w.e2, tp, e->conv2b, w.x, st))) return rc;
    if ((rc = launch_gelu_add(w.x, e->pos, (int64_t)tp * d, st))) return rc;
    for (int i = 0; i < e->n_layer; i++) {
        const wh_encoder::Block &b = e->blocks[i];
        // self-attention sub-layer (encoder.go:310-317, 340-379)
        if ((rc = launch_layernorm(w.x, b.ln1w, b.ln1b, w.xln, tp, d, st))) return rc;
        {
            // q, k and v of the same rows in one launch
            const DevMat *qkv[3] = {&b.q, &b.k, &b.v};
            const float *qkvb[3] = {b.qb, nullptr, b.vb};
            float *qkvo[3] = {w.q, w.k, w.v};
            if ((rc = launch_cross_gemm_n(qkv, 3, w.xln, tp, qkvb, qkvo, st))) return rc;
        }
        if ((rc = launch_enc_attn(w.q, w.k, w.v, tp, d, H, w.att, st))) return rc;
        if ((rc = launch_cross_gemm(b.o, w.att, tp, b.ob, w.x, st, 0, w.x))) return rc;
        // MLP sub-layer (encoder.go:319-325, 383-396)
        if ((rc = launch_layernorm(w.x, b.ln2w, b.ln2b, w.xln, tp, d, st))) return rc;
        if ((rc = launch_cross_gemm(b.fc1, w.xln, tp, b.fc1b, w.h, st, 1))) return rc;
        if ((rc = launch_cross_gemm(b.fc2, w.h, tp, b.fc2b, w.x, st, 0, w.x))) return rc;
        // encoder.go:327-329 checks the context after every block: with a flag
        // to poll, one block at a time is in flight
        if (cancel) {
            WH_HIP(hipStreamSynchronize(st));
            if (*cancel)
                return fail(WH_ERR_CANCELLED,
                            "model: encoder: cancelled after block " + std::to_string(i) + ": context canceled");
        }
    }
    if ((rc = launch_layernorm(w.x, e->lnw, e->lnb, out, tp, d, st))) return rc;
    WH_HIP(hipStreamSynchronize(st));
    return WH_OK;
}

// The stream and the workspace, made on the first encode of the handle.
int prepare(const wh_encoder *e, Work *w) {
    WH_HIP(hipSetDevice(e->device));
    if (!e->st) WH_HIP(hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking));
    if (!e->ws) WH_HIP(hipMalloc(&e->ws, carve(e, nullptr, w) * sizeof(float)));
    carve(e, e->ws, w);
    return WH_OK;
}

}  // namespace

// encoder.go:265-338 Encode: host mel in, host output out.
int encode(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out, int32_t out_cap,
           int32_t *out_rows, const volatile int32_t *cancel) {
    if (!e || !mel || !out || !out_rows) return fail(WH_ERR_INVALID, "model: encoder: null argument");
    *out_rows = 0;
    int rc, Tr;
    if ((rc = frames(e, n_mels, T, out_cap, &Tr))) return rc;
    // an already cancelled call stops where the reference's conv1 checks its context
    if (cancel && *cancel) return fail(WH_ERR_CANCELLED, "model: encoder: conv1: ml: conv1d: context canceled");
    std::lock_guard<std::mutex> lk(e->mu);
    Work w;
    if ((rc = prepare(e, &w))) return rc;
    const int tp = (Tr - 1) / 2 + 1;
    WH_HIP(hipMemcpyAsync(w.dmel, mel, sizeof(float) * e->n_mels * Tr, hipMemcpyHostToDevice, e->st));
    if ((rc = forward(e, w, w.dmel, Tr, w.xln, cancel))) return rc;
    WH_HIP(hipMemcpyAsync(out, w.xln, sizeof(float) * tp * e->n_state, hipMemcpyDeviceToHost, e->st));
    WH_HIP(hipStreamSynchronize(e->st));
    *out_rows = tp;
    return WH_OK;
}

// The same with mel and the output in device memory of the encoder's device.
int encode_device(const wh_encoder *e, const float *mel, int32_t n_mels, int32_t T, float *out, int32_t out_cap,
                  int32_t *out_rows, const volatile int32_t *cancel) {
    if (!e || !mel || !out || !out_rows) return fail(WH_ERR_INVALID, "model: encoder: null argument");
    *out_rows = 0;
    int rc, Tr;
    if ((rc = frames(e, n_mels, T, out_cap, &Tr))) return rc;
    if (cancel && *cancel) return fail(WH_ERR_CANCELLED, "model: encoder: conv1: ml: conv1d: context canceled");
    std::lock_guard<std::mutex> lk(e->mu);
    Work w;
    if ((rc = prepare(e, &w))) return rc;
    // mel rows stay T apart in the caller's buffer, except for the 2 n_ctx + 1
    // case, whose first n_mels * 2 n_ctx values are read as [n_mels, 2 n_ctx]
    if ((rc = forward(e, w, mel, Tr, out, cancel))) return rc;
    *out_rows = (Tr - 1) / 2 + 1;
    return WH_OK;
}

}  // namespace wh
