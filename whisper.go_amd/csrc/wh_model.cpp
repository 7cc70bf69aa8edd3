// Decoder model creation: tensor-name resolution, hyper-parameter inference
// and a one-time upload of every weight to HBM
// (internal/model/decoder.go:97-303, internal/model/compat.go:15-270).
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "wh_internal.h"
#include "wh_load.h"

namespace wh {
namespace mega {
int warm_decode(uint32_t type);
}
namespace batch {
int warm(uint32_t type, int d);
}
}  // namespace wh

namespace wh {

namespace {

// HF-style aliases of the encoder tensors (internal/model/compat.go:31-83).
std::string map_encoder_name(const std::string &name) {
    static const std::map<std::string, std::string> simple = {
        {"encoder.conv1.weight", "model.encoder.conv1.weight"},
        {"encoder.conv1.bias", "model.encoder.conv1.bias"},
        {"encoder.conv2.weight", "model.encoder.conv2.weight"},
        {"encoder.conv2.bias", "model.encoder.conv2.bias"},
        {"encoder.positional_embedding", "model.encoder.embed_positions.weight"},
        {"encoder.ln_post.weight", "model.encoder.layer_norm.weight"},
        {"encoder.ln_post.bias", "model.encoder.layer_norm.bias"},
    };
    auto it = simple.find(name);
    if (it != simple.end()) return it->second;
    static const std::string pre = "encoder.blocks.";
    if (name.compare(0, pre.size(), pre) != 0) return "";
    size_t dot = name.find('.', pre.size());
    if (dot == std::string::npos || dot == pre.size()) return "";
    const std::string idx = name.substr(pre.size(), dot - pre.size());
    for (char c : idx)
        if (c < '0' || c > '9') return "";
    static const std::map<std::string, std::string> suffix = {
        {"attn_ln.weight", "self_attn_layer_norm.weight"}, {"attn_ln.bias", "self_attn_layer_norm.bias"},
        {"attn.query.weight", "self_attn.q_proj.weight"},  {"attn.query.bias", "self_attn.q_proj.bias"},
        {"attn.key.weight", "self_attn.k_proj.weight"},    {"attn.value.weight", "self_attn.v_proj.weight"},
        {"attn.value.bias", "self_attn.v_proj.bias"},      {"attn.out.weight", "self_attn.out_proj.weight"},
        {"attn.out.bias", "self_attn.out_proj.bias"},      {"mlp_ln.weight", "final_layer_norm.weight"},
        {"mlp_ln.bias", "final_layer_norm.bias"},          {"mlp.0.weight", "fc1.weight"},
        {"mlp.0.bias", "fc1.bias"},                        {"mlp.2.weight", "fc2.weight"},
        {"mlp.2.bias", "fc2.bias"},
    };
    auto s = suffix.find(name.substr(dot + 1));
    if (s == suffix.end()) return "";
    return "model.encoder.layers." + idx + "." + s->second;
}

}  // namespace

// HF-style aliases of the decoder and encoder tensors (internal/model/compat.go:31-148).
std::string map_tensor_name(const std::string &name) {
    if (name.compare(0, 8, "encoder.") == 0) return map_encoder_name(name);
    static const std::map<std::string, std::string> simple = {
        {"decoder.token_embedding.weight", "model.decoder.embed_tokens.weight"},
        {"decoder.positional_embedding", "model.decoder.embed_positions.weight"},
        {"decoder.ln.weight", "model.decoder.layer_norm.weight"},
        {"decoder.ln.bias", "model.decoder.layer_norm.bias"},
    };
    auto it = simple.find(name);
    if (it != simple.end()) return it->second;
    static const std::string pre = "decoder.blocks.";
    if (name.compare(0, pre.size(), pre) != 0) return "";
    size_t dot = name.find('.', pre.size());
    if (dot == std::string::npos || dot == pre.size()) return "";
    const std::string idx = name.substr(pre.size(), dot - pre.size());
    for (char c : idx)
        if (c < '0' || c > '9') return "";
    static const std::map<std::string, std::string> suffix = {
        {"self_attn_ln.weight", "self_attn_layer_norm.weight"}, {"self_attn_ln.bias", "self_attn_layer_norm.bias"},
        {"self_attn.query.weight", "self_attn.q_proj.weight"},  {"self_attn.query.bias", "self_attn.q_proj.bias"},
        {"self_attn.key.weight", "self_attn.k_proj.weight"},    {"self_attn.value.weight", "self_attn.v_proj.weight"},
        {"self_attn.value.bias", "self_attn.v_proj.bias"},      {"self_attn.out.weight", "self_attn.out_proj.weight"},
        {"self_attn.out.bias", "self_attn.out_proj.bias"},      {"cross_attn_ln.weight", "encoder_attn_layer_norm.weight"},
        {"cross_attn_ln.bias", "encoder_attn_layer_norm.bias"}, {"cross_attn.query.weight", "encoder_attn.q_proj.weight"},
        {"cross_attn.query.bias", "encoder_attn.q_proj.bias"},  {"cross_attn.key.weight", "encoder_attn.k_proj.weight"},
        {"cross_attn.value.weight", "encoder_attn.v_proj.weight"}, {"cross_attn.value.bias", "encoder_attn.v_proj.bias"},
        {"cross_attn.out.weight", "encoder_attn.out_proj.weight"}, {"cross_attn.out.bias", "encoder_attn.out_proj.bias"},
        {"mlp_ln.weight", "final_layer_norm.weight"},           {"mlp_ln.bias", "final_layer_norm.bias"},
        {"mlp.0.weight", "fc1.weight"},                          {"mlp.0.bias", "fc1.bias"},
        {"mlp.2.weight", "fc2.weight"},                          {"mlp.2.bias", "fc2.bias"},
    };
    auto s = suffix.find(name.substr(dot + 1));
    if (s == suffix.end()) return "";
    return "model.decoder.layers." + idx + "." + s->second;
}

const wh_tensor *Table::resolve(const std::string &name) const {  // compat.go:15-29
    auto it = byname.find(name);
    if (it != byname.end()) return it->second;
    std::string alt = map_tensor_name(name);
    if (alt.empty()) return nullptr;
    it = byname.find(alt);
    return it == byname.end() ? nullptr : it->second;
}

uint64_t numel(const wh_tensor *t) {
    uint64_t n = 1;
    for (uint32_t i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}

int not_found(const std::string &name) {
    return fail(WH_ERR_NOT_FOUND, "model: load tensor \"" + name + "\": not found");
}

// gguf File.Tensor(): dequantise any stored type to float32.
int load_f32(const wh_tensor *t, std::vector<float> &out) {
    const uint64_t n = numel(t);
    const uint64_t need = gguf_row_bytes(t->type, n);
    if (need == 0 && n != 0) return fail(WH_ERR_UNSUPPORTED, "unsupported dtype: " + std::to_string(t->type));
    if (t->nbytes < need) return fail(WH_ERR_INVALID, std::string("gguf: tensor \"") + t->name + "\": short data");
    out.resize(n);
    return dequantize_host(t->type, (const uint8_t *)t->data, n, out.data());
}

int VecArena::add(const std::vector<float> &v, float **slot) {
    size_t off = host.size();
    host.insert(host.end(), v.begin(), v.end());
    while (host.size() % 64) host.push_back(0.0f);  // 256-byte alignment per vector
    fix.emplace_back(slot, off);
    return WH_OK;
}

// internal/model/compat.go:247-270 loadMatWeightAuto: a quantised 2-D tensor
// of the wanted shape is uploaded as is; anything else is dequantised to f32
// (transposed when stored [cols, rows]).
int load_matrix(const Table &tab, const std::string &name, int rows, int cols, DevMat &m) {
    const wh_tensor *t = tab.resolve(name);
    if (!t) return not_found(name);
    if (t->ndim == 2 && is_quant_type(t->type) && (int64_t)t->shape[0] == rows && (int64_t)t->shape[1] == cols) {
        int rc = devmat_plan(m, t->type, rows, cols);
        if (rc) return rc;
        return devmat_upload_typed(m, t->type, (const uint8_t *)t->data, t->nbytes);
    }
    if (t->ndim != 2) return fail(WH_ERR_INVALID, "model: invalid " + name + " shape");
    std::vector<float> f;
    int rc = load_f32(t, f);
    if (rc) return rc;
    if ((int64_t)t->shape[0] == rows && (int64_t)t->shape[1] == cols) {
        // as stored
    } else if ((int64_t)t->shape[0] == cols && (int64_t)t->shape[1] == rows) {
        std::vector<float> tr((size_t)rows * cols);
        for (int i = 0; i < cols; i++)
            for (int j = 0; j < rows; j++) tr[(size_t)j * cols + i] = f[(size_t)i * rows + j];
        f.swap(tr);
    } else {
        return fail(WH_ERR_INVALID, "model: unsupported " + name + " shape");
    }
    rc = devmat_plan(m, WH_TYPE_F32, rows, cols);
    if (rc) return rc;
    return devmat_upload_typed(m, WH_TYPE_F32, (const uint8_t *)f.data(), f.size() * 4);
}

// Float vectors (LN gains/biases, projection biases). The reference indexes them
// up to the layer width without a check; here a short vector is a load error.
int load_vector(const Table &tab, const std::string &name, VecArena &arena, float **slot, size_t min_len) {
    const wh_tensor *t = tab.resolve(name);
    if (!t) return not_found(name);
    std::vector<float> f;
    int rc = load_f32(t, f);
    if (rc) return rc;
    if (f.size() < min_len)
        return fail(WH_ERR_INVALID, "model: invalid " + name + " length " + std::to_string(f.size()) + ", want " +
                                        std::to_string(min_len));
    return arena.add(f, slot);
}

namespace {

// Row constants of a LayerNorm folded into the matrix w that reads its output:
// c = w·g (g the LayerNorm weight) and e = w·b + bias, by the quantised GEMV.
int fold_rows(const DevMat &w, const float *g, const float *b, const float *bias, int d, float *c, float *e) {
    const DevMat *mat = &w;
    GemvIn in{g, d};
    GemvOut out;
    out.y = c;
    out.ldy = w.rows;
    int rc = launch_gemv(&mat, &in, &out, 1, 1, nullptr);
    if (rc) return rc;
    GemvIn in2{b, d};
    GemvOut out2;
    out2.y = e;
    out2.ldy = w.rows;
    out2.bias = bias;
    return launch_gemv(&mat, &in2, &out2, 1, 1, nullptr);
}

// The folded LayerNorm constants of LN2 (cross query rows) and LN3 (fc1 rows)
// of every layer, when those matrices are quantised (the persistent decode
// kernel's condition); computed once at load.
int fold_layernorms(wh_model &m) {
    const int d = m.n_state;
    for (const Layer &l : m.layers)
        if (!is_quant_type(l.cq.type) || !is_quant_type(l.fc1.type)) return WH_OK;
    const size_t per = 2 * (size_t)d + 2 * 4 * (size_t)d;
    WH_HIP(hipMalloc(&m.fold_alloc, per * m.layers.size() * sizeof(float)));
    for (size_t i = 0; i < m.layers.size(); i++) {
        Layer &l = m.layers[i];
        float *base = (float *)m.fold_alloc + per * i;
        l.cqc = base;
        l.cqe = base + d;
        l.f1c = base + 2 * d;
        l.f1e = base + 6 * d;
        int rc;
        if ((rc = fold_rows(l.cq, l.ln2w, l.ln2b, l.cqb, d, l.cqc, l.cqe))) return rc;
        if ((rc = fold_rows(l.fc1, l.ln3w, l.ln3b, l.fc1b, d, l.f1c, l.f1e))) return rc;
    }
    WH_HIP(hipDeviceSynchronize());
    return WH_OK;
}

}  // namespace

void model_free(wh_model *m) {
    if (!m) return;
    devmat_free(m->tok);
    for (auto &l : m->layers) {
        DevMat *ms[] = {&l.sq, &l.sk, &l.sv, &l.so, &l.cq, &l.ck, &l.cv, &l.co, &l.fc1, &l.fc2, &l.sqkv};
        for (DevMat *d : ms) devmat_free(*d);
    }
    if (m->vec_alloc) (void)hipFree(m->vec_alloc);
    if (m->fold_alloc) (void)hipFree(m->fold_alloc);
    delete m;
}

int model_create(const wh_tensor *tensors, int32_t n, const wh_meta *meta, int32_t device, wh_model **out) {
    if (!out) return fail(WH_ERR_INVALID, "model: decoder: null output handle");
    *out = nullptr;
    if (n < 0 || (n > 0 && !tensors)) return fail(WH_ERR_INVALID, "model: decoder: invalid tensor table");
    Table tab;
    for (int32_t i = 0; i < n; i++) {
        if (!tensors[i].name) return fail(WH_ERR_INVALID, "model: decoder: tensor without a name");
        if (tensors[i].ndim > 4) return fail(WH_ERR_INVALID, std::string("model: decoder: too many dims for ") + tensors[i].name);
        tab.byname[tensors[i].name] = &tensors[i];
    }
    uint32_t n_head = meta ? meta->n_head : 0, n_layer = meta ? meta->n_layer : 0, n_ctx = meta ? meta->n_ctx : 0;
    uint32_t n_state = meta ? meta->n_state : 0, n_vocab = meta ? meta->n_vocab : 0;
    // decoder.go:107-164
    if (n_layer == 0) {
        uint32_t c = 0;
        while (tab.resolve("decoder.blocks." + std::to_string(c) + ".self_attn.query.weight")) c++;
        n_layer = c;
    }
    if (const wh_tensor *aq = tab.resolve("decoder.blocks.0.self_attn.query.weight"))
        if (aq->ndim == 2 && aq->shape[0] == aq->shape[1] && aq->shape[0] > 0) n_state = (uint32_t)aq->shape[0];
    if (n_ctx == 0 || n_state == 0) {
        const wh_tensor *p = tab.resolve("decoder.positional_embedding");
        if (!p) return not_found("decoder.positional_embedding");
        if (p->ndim != 2) return fail(WH_ERR_INVALID, "model: decoder: invalid positional embedding shape");
        if (n_state > 0) {
            if (p->shape[0] == n_state && p->shape[1] != n_state) n_ctx = (uint32_t)p->shape[1];
            else if (p->shape[1] == n_state) n_ctx = (uint32_t)p->shape[0];
        } else {
            n_ctx = (uint32_t)p->shape[0];
            n_state = (uint32_t)p->shape[1];
        }
    }
    if (n_vocab == 0) {
        const wh_tensor *e = tab.resolve("decoder.token_embedding.weight");
        if (!e) return not_found("decoder.token_embedding.weight");
        if (e->ndim != 2) return fail(WH_ERR_INVALID, "model: decoder: invalid token embedding shape");
        if (n_state > 0) {
            if (e->shape[1] == n_state) n_vocab = (uint32_t)e->shape[0];
            else if (e->shape[0] == n_state) n_vocab = (uint32_t)e->shape[1];
        } else {
            n_vocab = (uint32_t)e->shape[0];
            n_state = (uint32_t)e->shape[1];
        }
    }
    if (n_head == 0) {
        if (n_state % 64 != 0)
            return fail(WH_ERR_INVALID, "model: decoder: cannot infer head count from embedding length " + std::to_string(n_state));
        n_head = n_state / 64;
    }
    if (n_state == 0 || n_vocab == 0 || n_ctx == 0 || n_head == 0 || n_state % n_head != 0)
        return fail(WH_ERR_INVALID, "model: decoder: inconsistent hyper-parameters");

    WH_HIP(hipSetDevice(device));
    std::unique_ptr<wh_model, void (*)(wh_model *)> m(new wh_model(), model_free);
    m->device = device;
    m->n_vocab = (int32_t)n_vocab;
    m->n_state = (int32_t)n_state;
    m->n_head = (int32_t)n_head;
    m->n_layer = (int32_t)n_layer;
    m->n_ctx = (int32_t)n_ctx;
    const int d = m->n_state;
    int rc;
    // token embedding (decoder.go:176-189): quantised [n_vocab, d] stays quantised
    // (it is also the tied logits matrix); otherwise float, transposed if [d, n_vocab].
    {
        const wh_tensor *te = tab.resolve("decoder.token_embedding.weight");
        if (!te) return not_found("decoder.token_embedding.weight");
        if (te->ndim == 2 && is_quant_type(te->type) && (int64_t)te->shape[0] == m->n_vocab && (int64_t)te->shape[1] == d) {
            rc = devmat_plan(m->tok, te->type, m->n_vocab, d);
            if (!rc) rc = devmat_upload_typed(m->tok, te->type, (const uint8_t *)te->data, te->nbytes);
        } else {
            rc = load_matrix(tab, "decoder.token_embedding.weight", m->n_vocab, d, m->tok);
        }
        if (rc) return rc;
    }
    VecArena arena;
    {
        const wh_tensor *pe = tab.resolve("decoder.positional_embedding");
        if (!pe) return not_found("decoder.positional_embedding");
        if (pe->ndim != 2) return fail(WH_ERR_INVALID, "model: decoder: invalid positional embedding shape");
        std::vector<float> f;
        rc = load_f32(pe, f);
        if (rc) return rc;
        if ((int64_t)pe->shape[0] == d && (int64_t)pe->shape[1] == m->n_ctx) {
            std::vector<float> tr(f.size());
            for (int i = 0; i < d; i++)
                for (int j = 0; j < m->n_ctx; j++) tr[(size_t)j * d + i] = f[(size_t)i * m->n_ctx + j];
            f.swap(tr);
        }
        if (f.size() < (size_t)m->n_ctx * d) return fail(WH_ERR_INVALID, "model: decoder: positional embedding too small");
        arena.add(f, &m->pos);
    }
    m->layers.resize(n_layer);
    for (uint32_t i = 0; i < n_layer; i++) {
        Layer &l = m->layers[i];
        std::memset((void *)&l, 0, sizeof(float *) * 14);
        const std::string p = "decoder.blocks." + std::to_string(i) + ".";
        struct V { const char *suf; float **slot; } vecs[] = {
            {"self_attn_ln.weight", &l.ln1w}, {"self_attn_ln.bias", &l.ln1b}, {"self_attn.query.bias", &l.sqb},
            {"self_attn.value.bias", &l.svb}, {"self_attn.out.bias", &l.sob}, {"cross_attn_ln.weight", &l.ln2w},
            {"cross_attn_ln.bias", &l.ln2b}, {"cross_attn.query.bias", &l.cqb}, {"cross_attn.value.bias", &l.cvb},
            {"cross_attn.out.bias", &l.cob}, {"mlp_ln.weight", &l.ln3w}, {"mlp_ln.bias", &l.ln3b},
            {"mlp.0.bias", &l.fc1b}, {"mlp.2.bias", &l.fc2b}};
        for (auto &v : vecs)
            if ((rc = load_vector(tab, p + v.suf, arena, v.slot, v.slot == &l.fc1b ? 4 * (size_t)d : (size_t)d)))
                return rc;
        struct M { const char *suf; DevMat *mat; int rows, cols; } mats[] = {
            {"self_attn.query.weight", &l.sq, d, d}, {"self_attn.key.weight", &l.sk, d, d},
            {"self_attn.value.weight", &l.sv, d, d}, {"self_attn.out.weight", &l.so, d, d},
            {"cross_attn.query.weight", &l.cq, d, d}, {"cross_attn.key.weight", &l.ck, d, d},
            {"cross_attn.value.weight", &l.cv, d, d}, {"cross_attn.out.weight", &l.co, d, d},
            {"mlp.0.weight", &l.fc1, 4 * d, d},       {"mlp.2.weight", &l.fc2, d, 4 * d}};
        for (auto &mm : mats)
            if ((rc = load_matrix(tab, p + mm.suf, mm.rows, mm.cols, *mm.mat))) return rc;
        if (is_quant_type(l.sq.type) && l.sq.type == l.sk.type && l.sk.type == l.sv.type)
            if ((rc = devmat_stack({&l.sq, &l.sk, &l.sv}, l.sqkv))) return rc;
    }
    if ((rc = load_vector(tab, "decoder.ln.weight", arena, &m->lnw, (size_t)d))) return rc;
    if ((rc = load_vector(tab, "decoder.ln.bias", arena, &m->lnb, (size_t)d))) return rc;
    WH_HIP(hipMalloc(&m->vec_alloc, arena.host.size() * sizeof(float) + 256));
    WH_HIP(hipMemcpy(m->vec_alloc, arena.host.data(), arena.host.size() * sizeof(float), hipMemcpyHostToDevice));
    for (auto &f : arena.fix) *f.first = (float *)m->vec_alloc + f.second;
    if ((rc = fold_layernorms(*m))) return rc;
    // algorithmic weight bytes per token: every matrix once + the tied logits matrix
    uint64_t wb = m->tok.algo_bytes;
    for (auto &l : m->layers) {
        const DevMat *ms[] = {&l.sq, &l.sk, &l.sv, &l.so, &l.cq, &l.co, &l.fc1, &l.fc2};
        for (const DevMat *x : ms) wb += x->algo_bytes;
    }
    m->weight_bytes = wb;
    // load the persistent kernels' code objects now rather than in the first step
    if ((rc = mega::warm_decode(m->tok.type)) || (rc = batch::warm(m->tok.type, d))) return rc;
    {
        // the runtime sets up a stream's hardware queue on first use (~3 ms of the
        // first sequence's setup otherwise); it keeps it for the next stream
        hipStream_t st = nullptr;
        WH_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        WH_HIP(hipStreamDestroy(st));
    }
    *out = m.release();
    return WH_OK;
}

}  // namespace wh
