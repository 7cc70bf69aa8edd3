// Decoder state in HBM and the token loop on the host
// (internal/model/decoder.go:306-386 state, :413-525 greedy, :528-742 beam,
// :745-993 forward). Only token ids (and, in parity mode, logits) cross PCIe.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "wh_batch.h"
#include "wh_internal.h"
#include "wh_mega.h"

namespace wh {
namespace mega {
int launch_decode(uint32_t type, int grid, const MegaArgs &a, hipStream_t st);
}
namespace batch {
int launch(uint32_t type, int grid, const BArgs &a, hipStream_t st);
}

__global__ void k_zero_rows(float *base, size_t stride, int count, int len) {
    for (int r = blockIdx.x; r < count; r += gridDim.x)
        for (int j = threadIdx.x; j < len; j += blockDim.x) base[(size_t)r * stride + j] = 0.0f;
}

}  // namespace wh

struct wh_seq {
    const wh_model *m = nullptr;
    int S = 0, enc_len = 0, n_enc = 0, hist_cap = 0;
    hipStream_t st = nullptr;
    std::vector<void *> allocs;
    float *x = nullptr, *xln = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *h = nullptr;
    float *logits = nullptr;
    wh::GemvWork gw{};  // split-K workspace of the batched GEMV (6..16 streams)
    float *kv = nullptr;
    size_t kv_stream = 0, kv_layer = 0;  // floats
    float *crossK = nullptr, *crossV = nullptr;
    const float **kbase = nullptr, **vbase = nullptr;  // [L][S] device pointer tables
    wh::CrossBufs cb{};
    wh::SampleBufs sb{};
    int32_t *hist = nullptr, *hist_len = nullptr, *tok = nullptr, *pos = nullptr, *active = nullptr;
    int32_t *out_ids = nullptr, *topk_tok = nullptr;
    float *topk_lp = nullptr, *topk_logz = nullptr, *topk_part = nullptr;
    std::vector<int32_t> h_len;     // host mirror of hist_len
    std::vector<int32_t> h_active;  // host mirror of active
    std::vector<std::vector<int32_t>> h_hist;  // host mirror of the histories
    std::vector<float> h_inv, h_nst;  // host mirrors of the per-stream sampling parameters
    std::vector<int32_t> h_supp;
    int32_t *pinned_ids = nullptr;

    // persistent decode kernel (one stream, reference mask, uniform weight type)
    bool mega_ok = false;
    int mega_grid = 0;
    uint32_t mega_type = 0;
    unsigned mega_g = 0;
    int64_t mega_launches = 0;
    wh::mega::MegaArgs mega{};
    int32_t *mega_state = nullptr;  // pinned host copy of state_out

    // batched persistent forward (2..8 streams, reference mask, one quantised type)
    bool batch_ok = false;
    int batch_grid = 0;
    uint32_t batch_type = 0;
    int64_t batch_launches = 0;
    wh::batch::BArgs bargs{};
    unsigned *batch_errp = nullptr;  // pinned copy of the kernel's error word
    bool batch_pending = false;      // a copy of it is queued since the last check

    // optional per-kernel timing: an event pair around every launch
    struct ProfCat {
        std::string name;
        double ms = 0, bytes = 0;
        int64_t launches = 0;
    };
    struct Pending {
        hipEvent_t a, b;
        int cat;
        double bytes;
    };
    bool prof = false;
    std::vector<ProfCat> prof_cats;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_next = 0;
    hipEvent_t ev_get() {
        if (ev_next == ev_pool.size()) {
            hipEvent_t e;
            if (hipEventCreate(&e) != hipSuccess) return nullptr;
            ev_pool.push_back(e);
        }
        return ev_pool[ev_next++];
    }
    int cat_of(const char *name) {
        for (size_t i = 0; i < prof_cats.size(); i++)
            if (prof_cats[i].name == name) return (int)i;
        prof_cats.push_back(ProfCat{name});
        return (int)prof_cats.size() - 1;
    }
    void prof_resolve() {
        for (auto &p : pending) {
            float ms = 0;
            if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
                prof_cats[p.cat].ms += ms;
                prof_cats[p.cat].launches++;
                prof_cats[p.cat].bytes += p.bytes;
            }
        }
        pending.clear();
        ev_next = 0;
    }

    ~wh_seq() {
        if (st) (void)hipStreamSynchronize(st);
        for (hipEvent_t e : ev_pool) (void)hipEventDestroy(e);
        for (void *p : allocs) (void)hipFree(p);
        if (pinned_ids) (void)hipHostFree(pinned_ids);
        if (mega_state) (void)hipHostFree(mega_state);
        if (batch_errp) (void)hipHostFree(batch_errp);
        if (st) (void)hipStreamDestroy(st);
    }
    template <typename T>
    int alloc(T **p, size_t count) {
        void *d = nullptr;
        size_t bytes = std::max<size_t>(count * sizeof(T), 256);
        hipError_t e = hipMalloc(&d, bytes);
        if (e != hipSuccess) return wh::fail(WH_ERR_NOMEM, std::string("hip: alloc: ") + hipGetErrorString(e));
        allocs.push_back(d);
        *p = (T *)d;
        return WH_OK;
    }
};

namespace wh {

namespace {

constexpr int SAMPLE_PARTS = 64;

// Records an event pair around the launches in its scope when profiling is on;
// `bytes` is the algorithmic HBM traffic of the launch.
struct Prof {
    wh_seq &s;
    int cat = -1;
    double bytes;
    hipEvent_t a = nullptr;
    Prof(wh_seq &s_, const char *name, double b) : s(s_), bytes(b) {
        if (!s.prof) return;
        cat = s.cat_of(name);
        a = s.ev_get();
        if (a) (void)hipEventRecord(a, s.st);
    }
    ~Prof() {
        if (!s.prof || !a) return;
        hipEvent_t b = s.ev_get();
        if (!b) return;
        (void)hipEventRecord(b, s.st);
        s.pending.push_back({a, b, cat, bytes});
    }
};

double mat_bytes(const DevMat &m) { return (double)m.algo_bytes; }

// One step's forward of every active stream in the batched persistent kernel.
int batch_forward(wh_seq &s) {
    int rc;
    {
        Prof p(s, "forward_batch", (double)s.m->weight_bytes);
        if ((rc = batch::launch(s.batch_type, s.batch_grid, s.bargs, s.st))) return rc;
    }
    s.batch_launches++;
    WH_HIP(hipMemcpyAsync(s.batch_errp, s.bargs.err, sizeof(unsigned), hipMemcpyDeviceToHost, s.st));
    s.batch_pending = true;
    return WH_OK;
}

// After the caller's stream synchronisation: a batched forward whose wait gave up
// fails the step and turns the path off for this sequence.
int batch_check(wh_seq &s) {
    if (!s.batch_pending) return WH_OK;
    s.batch_pending = false;
    if (*s.batch_errp == 0) return WH_OK;
    s.batch_ok = false;
    (void)hipMemsetAsync(s.bargs.err, 0, sizeof(unsigned), s.st);
    (void)hipStreamSynchronize(s.st);
    return fail(WH_ERR_HIP, "batched persistent forward: a workgroup wait timed out");
}

int seq_forward(wh_seq &s) {
    if (s.batch_ok && s.m->attn_mode == 0) return batch_forward(s);
    const wh_model &m = *s.m;
    const int S = s.S, d = m.n_state, H = m.n_head, hd = d / H, ctx = m.n_ctx;
    hipStream_t st = s.st;
    int active = 0;
    for (int i = 0; i < S; i++) active += s.h_active[i] != 0;
    const double cross_kv_bytes = (double)active * s.enc_len * d * 4;  // one of K or V, per layer
    int rc;
    auto gemv1 = [&](const DevMat &w, const float *x, int ldx, float *y, int ldy, const float *bias, const float *res,
                     int gelu) {
        const DevMat *mat = &w;
        GemvIn in{x, ldx};
        GemvOut out;
        out.y = y; out.ldy = ldy; out.bias = bias; out.res = res; out.ldres = ldy; out.gelu = gelu;
        Prof p(s, "gemv", mat_bytes(w));
        return launch_gemv(&mat, &in, &out, 1, S, st, &s.gw);
    };
    {
        Prof p(s, "embed", 0);
        if ((rc = launch_embed(m, s.tok, s.pos, s.active, s.x, S, st))) return rc;
    }
    for (int li = 0; li < m.n_layer; li++) {
        const Layer &l = m.layers[li];
        // self-attention sub-layer (decoder.go:780-790, :836-908)
        {
            Prof p(s, "layernorm", 0);
            if ((rc = launch_layernorm(s.x, l.ln1w, l.ln1b, s.xln, S, d, st))) return rc;
        }
        if (l.sq.type == l.sk.type && l.sk.type == l.sv.type) {
            const DevMat *mats[3] = {&l.sq, &l.sk, &l.sv};
            GemvIn in[3] = {{s.xln, d}, {s.xln, d}, {s.xln, d}};
            GemvOut out[3];
            out[0].y = s.q; out[0].ldy = d; out[0].bias = l.sqb;
            out[1].y = s.k; out[1].ldy = d;
            out[2].y = s.v; out[2].ldy = d; out[2].bias = l.svb;
            Prof p(s, "gemv", mat_bytes(l.sq) + mat_bytes(l.sk) + mat_bytes(l.sv));
            if ((rc = launch_gemv(mats, in, out, 3, S, st, &s.gw))) return rc;
        } else {
            if ((rc = gemv1(l.sq, s.xln, d, s.q, d, l.sqb, nullptr, 0))) return rc;
            if ((rc = gemv1(l.sk, s.xln, d, s.k, d, nullptr, nullptr, 0))) return rc;
            if ((rc = gemv1(l.sv, s.xln, d, s.v, d, l.svb, nullptr, 0))) return rc;
        }
        {
            Prof p(s, "self_attn", 0);
            if ((rc = launch_self_attn(s.q, s.k, s.v, s.kv + (size_t)li * s.kv_layer, s.kv_stream, s.pos, s.active,
                                       s.attn, S, H, hd, ctx, m.attn_mode, st)))
                return rc;
        }
        if ((rc = gemv1(l.so, s.attn, d, s.x, d, l.sob, s.x, 0))) return rc;
        // cross-attention sub-layer (decoder.go:792-801, :911-971)
        {
            Prof p(s, "layernorm", 0);
            if ((rc = launch_layernorm(s.x, l.ln2w, l.ln2b, s.xln, S, d, st))) return rc;
        }
        if ((rc = gemv1(l.cq, s.xln, d, s.q, d, l.cqb, nullptr, 0))) return rc;
        {
            Prof p(s, "cross_attn", 2 * cross_kv_bytes);
            if ((rc = launch_cross_attn(s.q, s.kbase + (size_t)li * S, s.vbase + (size_t)li * S, s.active, s.attn, S, H,
                                        hd, s.enc_len, s.cb, st)))
                return rc;
        }
        if ((rc = gemv1(l.co, s.attn, d, s.x, d, l.cob, s.x, 0))) return rc;
        // MLP sub-layer (decoder.go:803-810, :974-993)
        {
            Prof p(s, "layernorm", 0);
            if ((rc = launch_layernorm(s.x, l.ln3w, l.ln3b, s.xln, S, d, st))) return rc;
        }
        if ((rc = gemv1(l.fc1, s.xln, d, s.h, 4 * d, l.fc1b, nullptr, 1))) return rc;
        if ((rc = gemv1(l.fc2, s.h, 4 * d, s.x, d, l.fc2b, s.x, 0))) return rc;
    }
    // final LN + tied logits (decoder.go:817-832)
    {
        Prof p(s, "layernorm", 0);
        if ((rc = launch_layernorm(s.x, m.lnw, m.lnb, s.xln, S, d, st))) return rc;
    }
    return gemv1(m.tok, s.xln, d, s.logits, m.n_vocab, nullptr, nullptr, 0);
}

int check_positions(const wh_seq &s) {
    for (int i = 0; i < s.S; i++) {
        if (!s.h_active[i]) continue;
        if (s.h_len[i] <= 0) return fail(WH_ERR_INVALID, "model: decode: forward: no tokens in state");
        if (s.h_len[i] - 1 >= s.m->n_ctx)
            return fail(WH_ERR_INVALID, "model: decode: forward: position " + std::to_string(s.h_len[i] - 1) +
                                            " >= context length " + std::to_string(s.m->n_ctx));
        if (s.h_len[i] + 1 > s.hist_cap) return fail(WH_ERR_INVALID, "model: decode: history capacity exceeded");
    }
    return WH_OK;
}

MatView view(const DevMat &m) {
    MatView v;
    v.qs = (const uint8_t *)m.qs;
    v.sc = m.sc;
    v.qh = m.qh;
    v.rows = m.rows;
    v.cols = m.cols;
    v.nb = m.nb;
    return v;
}

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

// Set up the persistent decode kernel for a one-stream sequence when the model
// fits its shape limits; otherwise the multi-kernel path serves every step.
int mega_setup(wh_seq &s) {
    const wh_model &m = *s.m;
    s.mega_ok = false;
    if (s.S != 1 || !env_int("WHISPER_HIP_PERSISTENT", 1)) return WH_OK;
    const int d = m.n_state, H = m.n_head, L = m.n_layer;
    if (d / H != 64 || d % 64 != 0 || !is_quant_type(m.tok.type)) return WH_OK;
    for (const Layer &l : m.layers) {
        if (!l.sqkv.alloc) return WH_OK;  // q, k, v not stacked (mixed types)
        if (!l.cqc || !l.f1c) return WH_OK;  // no folded LayerNorm constants
        const DevMat *ms[] = {&l.sqkv, &l.so, &l.cq, &l.co, &l.fc1, &l.fc2};
        for (const DevMat *x : ms)
            if (x->type != m.tok.type) return WH_OK;
    }
    int dev_cus = 0, lds_max = 0;
    if (hipDeviceGetAttribute(&dev_cus, hipDeviceAttributeMultiprocessorCount, m.device) != hipSuccess) return WH_OK;
    if (hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, m.device) != hipSuccess)
        return WH_OK;
    const int W = std::min(env_int("WHISPER_HIP_GRID", dev_cus), dev_cus);
    // C >= CMIN chunks of at most CHUNK_MAX keys, enough that a chunk's share of its
    // head's 64 cross-query rows fits the flat split; the last chunk is not empty
    const int nbd = d / 32;
    int C = std::max(mega::CMIN, (s.enc_len + mega::CHUNK_MAX - 1) / mega::CHUNK_MAX);
    while (C < mega::CMAX && !(mega::flat_fits(64 / C, nbd, mega::FQ, mega::RQ) &&
                               mega::flat_fits((64 + C - 1) / C, nbd, mega::FQ, mega::RQ)))
        C++;
    const int chunk = (s.enc_len + C - 1) / C;
    if (s.enc_len < 16 || (C - 1) * chunk >= s.enc_len || chunk > mega::CHUNK_MAX || chunk > 128 * mega::PKQ)
        return WH_OK;
    const int items = H * C;
    // per-workgroup row capacities of the kernel's register slots (compute waves only)
    auto per = [&](int rows, int n) { return (rows + n - 1) / n; };
    const int NC = mega::CWAVES;
    // exchange loads: XS, XD, XH, XT, XP pairs per lane
    if (d > 64 * NC * mega::XS || d > 64 * mega::XD || 4 * d > 64 * NC * mega::XH || 4 * W > 64 * mega::XT ||
        mega::CMAX * 65 > 64 * mega::XP)
        return WH_OK;
    if (C > mega::CMAX || W < 8 || items >= W || W > 256 || H > 256 || per(d, W) > NC * mega::SD)
        return WH_OK;
    // flat splits: both row counts a workgroup (or item) can get
    auto flat2 = [&](int rows, int n, int nb, int P, int RS) {
        return mega::flat_fits(rows / n, nb, P, RS) && mega::flat_fits(per(rows, n), nb, P, RS);
    };
    if (!flat2(64, C, nbd, mega::FQ, mega::RQ) || !flat2(4 * d, W, nbd, mega::FE, mega::RE) ||
        !flat2(d, W, 4 * nbd, mega::FF, mega::RF))
        return WH_OK;
    if (mega::lds_bytes(d, L, m.n_vocab, W, chunk) + 64 > (size_t)lds_max) return WH_OK;
    auto fits32 = [](const DevMat &x) { return (uint64_t)x.rows * x.nb * 32 < (1ull << 32); };
    if (!fits32(m.tok)) return WH_OK;
    for (const Layer &l : m.layers)
        if (!fits32(l.sqkv) || !fits32(l.so) || !fits32(l.cq) || !fits32(l.co) || !fits32(l.fc1) || !fits32(l.fc2))
            return WH_OK;
    // Roles. Workgroup w runs on XCD w % 8; the chunks of one head go to one
    // XCD when they fit, so their head-local exchanges stay near one L2.
    std::vector<mega::Role> roles(W);
    for (auto &r : roles) r = mega::Role{-1, 0, 0, 0, 0, {0, 0, 0}};
    {
        std::vector<std::vector<int>> free_on(8);
        for (int w = 0; w < W; w++) free_on[w % 8].push_back(w);
        std::vector<size_t> used(8, 0);
        bool ok = true;
        for (int h = 0; h < H && ok; h++) {
            int x = h % 8;
            for (int k = 0; k < 8 && used[x] + C > free_on[x].size(); k++) x = (x + 1) % 8;
            if (used[x] + C > free_on[x].size()) ok = false;
            for (int c = 0; ok && c < C; c++) roles[free_on[x][used[x]++]].item = h * C + c;
        }
        if (!ok) {
            for (auto &r : roles) r.item = -1;
            for (int i = 0; i < items; i++) roles[i].item = i;
        }
    }
    // the side rows go to the workgroups without an item
    std::vector<int> side;
    for (int w = 0; w < W; w++)
        if (roles[w].item < 0) side.push_back(w);
    const int ns = (int)side.size();
    if (ns == 0 || per(3 * d, ns) > NC * mega::SQ || per(d, ns) > NC * mega::SO) return WH_OK;
    for (size_t j = 0; j < side.size(); j++) {
        const long n = (long)side.size();
        mega::Role &r = roles[side[j]];
        r.q0 = (int)(3L * d * j / n); r.q1 = (int)(3L * d * (j + 1) / n);
        r.o0 = (int)((long)d * j / n); r.o1 = (int)((long)d * (j + 1) / n);
    }
    mega::MegaArgs &a = s.mega;
    std::vector<mega::MegaLayer> ly(L);
    for (int li = 0; li < L; li++) {
        const Layer &l = m.layers[li];
        mega::MegaLayer &x = ly[li];
        x.sqkv = view(l.sqkv); x.so = view(l.so); x.cq = view(l.cq); x.co = view(l.co); x.fc1 = view(l.fc1);
        x.fc2 = view(l.fc2);
        x.ln1w = l.ln1w; x.ln1b = l.ln1b; x.svb = l.svb; x.sob = l.sob; x.ln2w = l.ln2w; x.ln2b = l.ln2b;
        x.cqb = l.cqb; x.cob = l.cob; x.ln3w = l.ln3w; x.ln3b = l.ln3b; x.fc1b = l.fc1b; x.fc2b = l.fc2b;
        x.cqc = l.cqc; x.cqe = l.cqe; x.f1c = l.f1c; x.f1e = l.f1e;
        x.crossK = s.crossK + (size_t)li * s.enc_len * d;
        x.crossV = s.crossV + (size_t)li * s.enc_len * d;
        x.kv = s.kv + (size_t)li * s.kv_layer;
    }
    int rc;
    mega::MegaLayer *dl = nullptr;
    if ((rc = s.alloc(&dl, (size_t)L))) return rc;
    WH_HIP(hipMemcpy(dl, ly.data(), sizeof(mega::MegaLayer) * L, hipMemcpyHostToDevice));
    a.layers = dl;
    mega::Role *droles = nullptr;
    if ((rc = s.alloc(&droles, (size_t)W))) return rc;
    WH_HIP(hipMemcpy(droles, roles.data(), sizeof(mega::Role) * W, hipMemcpyHostToDevice));
    a.roles = droles;
    a.L = L; a.d = d; a.H = H; a.ctx = m.n_ctx; a.V = m.n_vocab; a.enc_len = s.enc_len;
    a.C = C; a.chunk_len = chunk;
    a.scale = (float)(1.0 / sqrt(64.0));
    a.tok = view(m.tok);
    a.pos_emb = m.pos; a.lnw = m.lnw; a.lnb = m.lnb;
    a.hist = s.hist;
#define MALLOC(p, n) do { if ((rc = s.alloc(&(p), (n)))) return rc; } while (0)
    // exchange pairs start at phase 0; the kernel's phases count from g0 + 1
    const size_t npairs[] = {(size_t)d, (size_t)2 * d, (size_t)d, (size_t)4 * d, (size_t)d, (size_t)d, (size_t)items,
                             (size_t)items * 65, (size_t)W * 4, 1};
    uint64_t **pbuf[] = {&a.xg, &a.sa, &a.x2, &a.hbuf, &a.attn, &a.qx, &a.cmax, &a.parts, &a.part, &a.eot_logit};
    for (int i = 0; i < 10; i++) {
        MALLOC(*pbuf[i], npairs[i]);
        WH_HIP(hipMemsetAsync(*pbuf[i], 0, sizeof(uint64_t) * npairs[i], s.st));
    }
    MALLOC(a.err, 1); MALLOC(a.state_out, 4); MALLOC(a.out_tokens, (size_t)s.hist_cap);
#undef MALLOC
    WH_HIP(hipMemsetAsync(a.err, 0, sizeof(unsigned), s.st));
    WH_HIP(hipHostMalloc((void **)&s.mega_state, sizeof(int32_t) * 8, hipHostMallocDefault));
    WH_HIP(hipStreamSynchronize(s.st));
    s.mega_g = 0;
    s.mega_grid = W;
    s.mega_type = m.tok.type;
    s.mega_ok = true;
    return WH_OK;
}

// Set up the batched persistent forward for a sequence of 2..8 streams (2..16
// with WHISPER_HIP_BATCH=1; 0 turns it off) when the model fits it (head size 64,
// width <= 2048, every matrix of the token embedding's quantised type, q/k/v
// stacked); otherwise the multi-kernel chain serves the steps. Past 8 states the
// per-lane FMA work of the batched GEMV outgrows the chain's matrix-core GEMV on
// large models, so the chain is the default there.
int batch_setup(wh_seq &s) {
    const wh_model &m = *s.m;
    s.batch_ok = false;
    const int want = env_int("WHISPER_HIP_BATCH", -1);
    if (s.S < 2 || s.S > batch::SMAX || want == 0 || (want < 0 && s.S > 8)) return WH_OK;
    const int d = m.n_state, H = m.n_head, L = m.n_layer;
    if (d / H != 64 || d % 64 != 0 || d > 2048 || !is_quant_type(m.tok.type)) return WH_OK;
    for (const Layer &l : m.layers) {
        if (!l.sqkv.alloc) return WH_OK;
        const DevMat *ms[] = {&l.sqkv, &l.so, &l.cq, &l.co, &l.fc1, &l.fc2};
        for (const DevMat *x : ms)
            if (x->type != m.tok.type) return WH_OK;
    }
    int cus = 0, lds_max = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m.device) != hipSuccess) return WH_OK;
    if (hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, m.device) != hipSuccess)
        return WH_OK;
    const int W = std::min(env_int("WHISPER_HIP_GRID", cus), cus);
    // LDS for the staged [S][d] inputs and the LayerNorm weights; the fc2 column
    // passes keep a workgroup's rows within one pass
    // cross attention: every (state, head, key chunk) item has a workgroup, or one
    // chunk per head when the heads alone exceed the grid; a chunk's scores stay in LDS
    const int xchunks = std::min(std::max(1, W / (s.S * H)), batch::CMAX);
    if (W < 8 || (size_t)lds_max < batch::LDS_BYTES || (d + W - 1) / W > batch::pass_rows(d) || d > batch::LNMAX ||
        L > batch::LMAX ||
        s.S * (d / 32) > batch::XBUDGET / 128 ||
        (size_t)(s.enc_len + xchunks - 1) / xchunks * sizeof(float) > (size_t)batch::XBUDGET)
        return WH_OK;
    std::vector<batch::BLayer> ly(L);
    for (int li = 0; li < L; li++) {
        const Layer &l = m.layers[li];
        batch::BLayer &x = ly[li];
        x.sqkv = view(l.sqkv); x.so = view(l.so); x.cq = view(l.cq); x.co = view(l.co); x.fc1 = view(l.fc1);
        x.fc2 = view(l.fc2);
        x.ln1w = l.ln1w; x.ln1b = l.ln1b; x.svb = l.svb; x.sob = l.sob; x.ln2w = l.ln2w; x.ln2b = l.ln2b;
        x.cqb = l.cqb; x.cob = l.cob; x.ln3w = l.ln3w; x.ln3b = l.ln3b; x.fc1b = l.fc1b; x.fc2b = l.fc2b;
        x.kv = s.kv + (size_t)li * s.kv_layer;
        x.kbase = s.kbase + (size_t)li * s.S;
        x.vbase = s.vbase + (size_t)li * s.S;
    }
    int rc;
    batch::BLayer *dl = nullptr;
    if ((rc = s.alloc(&dl, (size_t)L))) return rc;
    WH_HIP(hipMemcpy(dl, ly.data(), sizeof(batch::BLayer) * L, hipMemcpyHostToDevice));
    batch::BArgs &a = s.bargs;
    a.layers = dl;
    a.L = L; a.d = d; a.H = H; a.ctx = m.n_ctx; a.V = m.n_vocab; a.enc_len = s.enc_len; a.S = s.S;
    a.xchunks = xchunks;
    a.kv_stream = s.kv_stream;
    a.tok = view(m.tok);
    a.pos_emb = m.pos; a.lnw = m.lnw; a.lnb = m.lnb;
    a.tokv = s.tok; a.posv = s.pos; a.active = s.active;
    a.logits = s.logits;
    // the exchanged {tag, value} pairs start with tag 0, below every phase's tag
    const size_t items = (size_t)s.S * H * xchunks, sd = (size_t)s.S * d;
    struct { uint64_t **p; size_t n; } pairs[] = {{&a.x, sd},      {&a.x2, sd},         {&a.q, sd},
                                                  {&a.h, 4 * sd},  {&a.attn, sd},       {&a.sa, (size_t)L * sd},
                                                  {&a.pv, items * 65}, {&a.xmax, items}};
    for (auto &b : pairs) {
        if ((rc = s.alloc(b.p, b.n))) return rc;
        WH_HIP(hipMemsetAsync(*b.p, 0, sizeof(uint64_t) * b.n, s.st));
    }
    if ((rc = s.alloc(&a.flags, (size_t)W)) || (rc = s.alloc(&a.err, 1))) return rc;
    WH_HIP(hipMemsetAsync(a.flags, 0, sizeof(unsigned) * W, s.st));
    WH_HIP(hipMemsetAsync(a.err, 0, sizeof(unsigned), s.st));
    a.scale = (float)(1.0 / sqrt(64.0));
    // GEMV rows on the matrix cores from 9 states (measured: 16 large-v3 Q4_1 streams
    // 2292 against 2172 tokens/s; beam 5 small Q5_1 1047 against 1305 steps/s);
    // WHISPER_HIP_BATCH_MFMA = 0 or 1 forces the choice
    {
        const int mf = env_int("WHISPER_HIP_BATCH_MFMA", -1);
        a.mfma = mf < 0 ? s.S >= 9 : mf != 0;
    }
    WH_HIP(hipHostMalloc((void **)&s.batch_errp, sizeof(unsigned), hipHostMallocDefault));
    *s.batch_errp = 0;
    WH_HIP(hipStreamSynchronize(s.st));
    s.batch_grid = W;
    s.batch_type = m.tok.type;
    s.batch_ok = true;
    return WH_OK;
}

// Run up to n greedy steps of stream 0 in the persistent kernel. Stops early on
// the reference's rules when stop_rules is set (EOT, > 20 repeats, max_len).
int mega_run(wh_seq &s, int n, float inv_temp, int suppress_nst, float nst, int max_len, int prev, int streak,
             float *out_logits, int32_t *out_ids, int *produced, int *prev_out, int *streak_out) {
    mega::MegaArgs a = s.mega;
    const std::vector<int32_t> &h = s.h_hist[0];
    a.tok0 = h.back();
    a.len0 = (int)h.size();
    a.prev0 = prev;
    a.streak0 = streak;
    a.n_steps = n;
    a.max_len = max_len;
    a.eot = s.m->eot;
    a.suppress_nst = suppress_nst;
    a.inv_temp = inv_temp;
    a.nst = nst;
    a.out_logits = out_logits ? s.logits : nullptr;
    a.g0 = s.mega_g;
    int rc;
    {
        Prof p(s, "decode_persistent", 0);  // algorithmic bytes set below, once the step count is known
        if ((rc = mega::launch_decode(s.mega_type, s.mega_grid, a, s.st))) return rc;
    }
    s.mega_launches++;
    WH_HIP(hipMemcpyAsync(s.mega_state, a.state_out, sizeof(int32_t) * 4, hipMemcpyDeviceToHost, s.st));
    WH_HIP(hipMemcpyAsync(s.mega_state + 4, a.err, sizeof(unsigned), hipMemcpyDeviceToHost, s.st));
    WH_HIP(hipStreamSynchronize(s.st));
    if (s.mega_state[4] != 0) {
        // a bounded wait expired: disable the path for this sequence
        s.mega_ok = false;
        (void)hipMemsetAsync(a.err, 0, sizeof(unsigned), s.st);
        (void)hipStreamSynchronize(s.st);
        return fail(WH_ERR_HIP, "persistent decode: a workgroup wait timed out");
    }
    const int got = s.mega_state[0];
    s.mega_g = (unsigned)s.mega_state[3];
    if (s.prof && !s.pending.empty()) {
        // quantised weight bytes of every step the launch ran (token rows included)
        s.pending.back().bytes = (double)s.m->weight_bytes * got;
        s.prof_resolve();
    }
    std::vector<int32_t> ids(std::max(got, 1));
    if (got > 0) WH_HIP(hipMemcpy(ids.data(), a.out_tokens, sizeof(int32_t) * got, hipMemcpyDeviceToHost));
    if (out_logits) WH_HIP(hipMemcpy(out_logits, s.logits, sizeof(float) * s.m->n_vocab, hipMemcpyDeviceToHost));
    for (int i = 0; i < got; i++) {
        s.h_hist[0].push_back(ids[i]);
        if (out_ids) out_ids[i] = ids[i];
    }
    s.h_len[0] = (int32_t)s.h_hist[0].size();
    // keep the multi-kernel path's device scalars in step
    int32_t meta[3] = {s.h_len[0], s.h_hist[0].back(), s.h_len[0] - 1};
    WH_HIP(hipMemcpy(s.hist_len, &meta[0], 4, hipMemcpyHostToDevice));
    WH_HIP(hipMemcpy(s.tok, &meta[1], 4, hipMemcpyHostToDevice));
    WH_HIP(hipMemcpy(s.pos, &meta[2], 4, hipMemcpyHostToDevice));
    *produced = got;
    if (prev_out) *prev_out = s.mega_state[1];
    if (streak_out) *streak_out = s.mega_state[2];
    return WH_OK;
}

// Per-stream sampling parameters for the sampling kernels; uploaded only when
// they change. Arrays of S entries.
int set_sample_params(wh_seq &s, const float *inv, const int32_t *supp, const float *nst) {
    bool same = true;
    for (int i = 0; i < s.S; i++)
        same &= s.h_inv[i] == inv[i] && s.h_supp[i] == (supp[i] != 0) && s.h_nst[i] == nst[i];
    if (same) return WH_OK;
    for (int i = 0; i < s.S; i++) {
        s.h_inv[i] = inv[i];
        s.h_supp[i] = supp[i] != 0;
        s.h_nst[i] = nst[i];
    }
    WH_HIP(hipMemcpyAsync(s.sb.inv_temp, s.h_inv.data(), sizeof(float) * s.S, hipMemcpyHostToDevice, s.st));
    WH_HIP(hipMemcpyAsync(s.sb.supp, s.h_supp.data(), sizeof(int32_t) * s.S, hipMemcpyHostToDevice, s.st));
    WH_HIP(hipMemcpyAsync(s.sb.nst, s.h_nst.data(), sizeof(float) * s.S, hipMemcpyHostToDevice, s.st));
    // the host vectors are the copies' sources: they must not change before the copies ran
    WH_HIP(hipStreamSynchronize(s.st));
    return WH_OK;
}

int set_sample_params_all(wh_seq &s, float inv, int32_t supp, float nst) {
    std::vector<float> a(s.S, inv), c(s.S, nst);
    std::vector<int32_t> b(s.S, supp);
    return set_sample_params(s, a.data(), b.data(), c.data());
}

int upload_active(wh_seq &s, const int32_t *active) {
    for (int i = 0; i < s.S; i++) s.h_active[i] = active ? (active[i] != 0) : 1;
    WH_HIP(hipMemcpyAsync(s.active, s.h_active.data(), sizeof(int32_t) * s.S, hipMemcpyHostToDevice, s.st));
    return WH_OK;
}

}  // namespace

// encs: host buffers, or (dev) device memory of the model's device, read in place
int seq_create(const wh_model *m, int32_t S, const float *const *encs, int32_t enc_len, int32_t enc_dim,
               int32_t shared, wh_seq **out, int32_t dev) {
    if (!m || !out) return fail(WH_ERR_INVALID, "seq: null argument");
    *out = nullptr;
    if (S < 1 || S > 16) return fail(WH_ERR_INVALID, "seq: n_streams must be in [1,16]");
    if (enc_dim != m->n_state || enc_len <= 0)
        return fail(WH_ERR_INVALID, "model: decoder: encoder output must be [T, " + std::to_string(m->n_state) +
                                        "], got [" + std::to_string(enc_len) + " " + std::to_string(enc_dim) + "]");
    if (!encs) return fail(WH_ERR_INVALID, "seq: null encoder outputs");
    WH_HIP(hipSetDevice(m->device));
    if (dev)
        for (int e = 0; e < (shared ? 1 : S); e++) {
            hipPointerAttribute_t at;
            const hipError_t pe = encs[e] ? hipPointerGetAttributes(&at, encs[e]) : hipErrorInvalidValue;
            if (pe != hipSuccess) (void)hipGetLastError();
            if (pe != hipSuccess || at.type != hipMemoryTypeDevice || at.device != m->device)
                return fail(WH_ERR_INVALID, "seq: encoder output " + std::to_string(e) +
                                                " is not device memory of the model's device");
        }
    std::unique_ptr<wh_seq> s(new wh_seq());
    s->m = m;
    s->S = S;
    s->enc_len = enc_len;
    s->n_enc = shared ? 1 : S;
    s->hist_cap = m->n_ctx + 64;
    WH_HIP(hipStreamCreateWithFlags(&s->st, hipStreamNonBlocking));
    const int d = m->n_state, H = m->n_head, hd = d / H, L = m->n_layer, V = m->n_vocab;
    int rc;
#define ALLOC(p, n) do { if ((rc = s->alloc(&(p), (n)))) return rc; } while (0)
    ALLOC(s->x, (size_t)S * d);
    ALLOC(s->xln, (size_t)S * d);
    ALLOC(s->q, (size_t)S * d);
    ALLOC(s->k, (size_t)S * d);
    ALLOC(s->v, (size_t)S * d);
    ALLOC(s->attn, (size_t)S * d);
    ALLOC(s->h, (size_t)S * 4 * d);
    ALLOC(s->logits, (size_t)S * V);
    s->kv_layer = (size_t)2 * H * m->n_ctx * hd;
    s->kv_stream = s->kv_layer * L;
    ALLOC(s->kv, s->kv_stream * S);
    WH_HIP(hipMemsetAsync(s->kv, 0, s->kv_stream * S * sizeof(float), s->st));
    const size_t cross_per = (size_t)L * enc_len * d;
    ALLOC(s->crossK, cross_per * s->n_enc);
    ALLOC(s->crossV, cross_per * s->n_enc);
    ALLOC(s->kbase, (size_t)L * S);
    ALLOC(s->vbase, (size_t)L * S);
    {
        std::vector<const float *> kb((size_t)L * S), vb((size_t)L * S);
        for (int li = 0; li < L; li++)
            for (int i = 0; i < S; i++) {
                const int e = shared ? 0 : i;
                kb[(size_t)li * S + i] = s->crossK + ((size_t)e * L + li) * enc_len * d;
                vb[(size_t)li * S + i] = s->crossV + ((size_t)e * L + li) * enc_len * d;
            }
        WH_HIP(hipMemcpy(s->kbase, kb.data(), kb.size() * sizeof(void *), hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(s->vbase, vb.data(), vb.size() * sizeof(void *), hipMemcpyHostToDevice));
    }
    s->cb.chunk_len = 128;
    s->cb.chunks = (enc_len + 127) / 128;
    ALLOC(s->cb.scores, (size_t)S * H * enc_len);
    ALLOC(s->cb.cmax, (size_t)S * H * s->cb.chunks);
    ALLOC(s->cb.pvt, (size_t)S * H * s->cb.chunks * 65);
    ALLOC(s->cb.cnt, (size_t)S * H);
    WH_HIP(hipMemsetAsync(s->cb.pvt, 0, sizeof(uint64_t) * S * H * s->cb.chunks * 65, s->st));
    WH_HIP(hipMemsetAsync(s->cb.cnt, 0, sizeof(uint32_t) * S * H, s->st));
    s->sb.parts = SAMPLE_PARTS;
    ALLOC(s->sb.cur, (size_t)S * V);
    ALLOC(s->sb.part_val, (size_t)S * SAMPLE_PARTS);
    ALLOC(s->sb.part_idx, (size_t)S * SAMPLE_PARTS);
    ALLOC(s->sb.part_val2, (size_t)S * SAMPLE_PARTS);
    ALLOC(s->sb.part_idx2, (size_t)S * SAMPLE_PARTS);
    ALLOC(s->sb.inv_temp, (size_t)S);
    ALLOC(s->sb.supp, (size_t)S);
    ALLOC(s->sb.nst, (size_t)S);
    ALLOC(s->hist, (size_t)S * s->hist_cap);
    ALLOC(s->hist_len, (size_t)S);
    ALLOC(s->tok, (size_t)S);
    ALLOC(s->pos, (size_t)S);
    ALLOC(s->active, (size_t)S);
    ALLOC(s->out_ids, (size_t)S);
    ALLOC(s->topk_tok, (size_t)S * 8);
    ALLOC(s->topk_lp, (size_t)S * 8);
    ALLOC(s->topk_logz, (size_t)S);
    ALLOC(s->topk_part, (size_t)TOPK_SCRATCH_FLOATS);
    if (S >= 6) {
        // split-K workspace of the batched GEMV
        s->gw.tiles = GEMVM_SPLIT_TILES;
        ALLOC(s->gw.part, (size_t)s->gw.tiles * GEMVM_MAX_SPLIT * 256);
        ALLOC(s->gw.cnt, (size_t)s->gw.tiles);
        WH_HIP(hipMemsetAsync(s->gw.part, 0, sizeof(uint64_t) * s->gw.tiles * GEMVM_MAX_SPLIT * 256, s->st));
        WH_HIP(hipMemsetAsync(s->gw.cnt, 0, sizeof(uint32_t) * s->gw.tiles, s->st));
    }
#undef ALLOC
    WH_HIP(hipMemsetAsync(s->hist_len, 0, sizeof(int32_t) * S, s->st));
    WH_HIP(hipMemsetAsync(s->tok, 0, sizeof(int32_t) * S, s->st));
    WH_HIP(hipMemsetAsync(s->pos, 0, sizeof(int32_t) * S, s->st));
    // pinned staging: ids/top-k tokens [16*8], top-k logprobs [16*8], log-normalisers [16]
    WH_HIP(hipHostMalloc((void **)&s->pinned_ids, sizeof(int32_t) * (16 * 8 * 2 + 16), hipHostMallocDefault));
    s->h_len.assign(S, 0);
    s->h_active.assign(S, 1);
    s->h_hist.assign(S, {});
    s->h_inv.assign(S, 1.0f);
    s->h_supp.assign(S, 0);
    s->h_nst.assign(S, 0.0f);
    {
        std::vector<int32_t> z(S, 0);
        std::vector<float> one(S, 1.0f), zf(S, 0.0f);
        WH_HIP(hipMemcpy(s->sb.inv_temp, one.data(), sizeof(float) * S, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(s->sb.supp, z.data(), sizeof(int32_t) * S, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(s->sb.nst, zf.data(), sizeof(float) * S, hipMemcpyHostToDevice));
    }
    // cross K/V projections of every encoder output (decoder.go:923-940), once per sequence
    float *stage = nullptr;  // host encoder outputs are uploaded here one at a time
    if (!dev) WH_HIP(hipMalloc(&stage, sizeof(float) * (size_t)enc_len * d));
    for (int e = 0; e < s->n_enc; e++) {
        if (!encs[e]) { (void)hipFree(stage); return fail(WH_ERR_INVALID, "seq: null encoder output"); }
        const float *enc = encs[e];
        if (!dev) {
            hipError_t he =
                hipMemcpyAsync(stage, encs[e], sizeof(float) * (size_t)enc_len * d, hipMemcpyHostToDevice, s->st);
            if (he != hipSuccess) { (void)hipFree(stage); return fail(WH_ERR_HIP, "hip: encoder upload failed"); }
            enc = stage;
        }
        for (int li = 0; li < L; li++) {
            const Layer &l = m->layers[li];
            float *K = s->crossK + ((size_t)e * L + li) * enc_len * d;
            float *Vv = s->crossV + ((size_t)e * L + li) * enc_len * d;
            // the layer's K and V in one launch
            const DevMat *kv[2] = {&l.ck, &l.cv};
            const float *kvb[2] = {nullptr, l.cvb};
            float *kvo[2] = {K, Vv};
            if ((rc = launch_cross_gemm_n(kv, 2, enc, enc_len, kvb, kvo, s->st))) {
                (void)hipStreamSynchronize(s->st);
                (void)hipFree(stage);
                return rc;
            }
        }
        if (!dev) (void)hipStreamSynchronize(s->st);  // the staging buffer is reused for the next stream
    }
    (void)hipFree(stage);
    WH_HIP(hipStreamSynchronize(s->st));
    if ((rc = mega_setup(*s))) return rc;
    if ((rc = batch_setup(*s))) return rc;
    *out = s.release();
    return WH_OK;
}

int seq_set_tokens(wh_seq *s, int32_t i, const int32_t *tokens, int32_t n, int32_t reset_kv) {
    if (!s || i < 0 || i >= s->S) return fail(WH_ERR_INVALID, "seq: stream index out of range");
    if (n < 0 || n > s->hist_cap - 1 || (n > 0 && !tokens)) return fail(WH_ERR_INVALID, "seq: invalid token history");
    for (int j = 0; j < n; j++)
        if (tokens[j] < 0 || tokens[j] >= s->m->n_vocab)
            return fail(WH_ERR_INVALID, "model: decode: forward: invalid token ID " + std::to_string(tokens[j]));
    WH_HIP(hipSetDevice(s->m->device));
    if (n > 0)
        WH_HIP(hipMemcpyAsync(s->hist + (size_t)i * s->hist_cap, tokens, sizeof(int32_t) * n, hipMemcpyHostToDevice, s->st));
    int32_t meta[3] = {n, n > 0 ? tokens[n - 1] : 0, n > 0 ? n - 1 : 0};
    // the three scalars are copied from a host array that outlives the call (synchronised below)
    WH_HIP(hipMemcpyAsync(s->hist_len + i, &meta[0], 4, hipMemcpyHostToDevice, s->st));
    WH_HIP(hipMemcpyAsync(s->tok + i, &meta[1], 4, hipMemcpyHostToDevice, s->st));
    WH_HIP(hipMemcpyAsync(s->pos + i, &meta[2], 4, hipMemcpyHostToDevice, s->st));
    if (reset_kv) {
        const wh_model &m = *s->m;
        float *base = s->kv + (size_t)i * s->kv_stream;
        if (m.attn_mode == 0) {
            // only cache row 0 is ever read under the reference mask: clear it in
            // every (layer, K/V plane, head)
            const int hd = m.n_state / m.n_head;
            const int count = m.n_layer * 2 * m.n_head;
            hipLaunchKernelGGL(k_zero_rows, dim3(std::min(count, 1024)), dim3(64), 0, s->st, base,
                               (size_t)m.n_ctx * hd, count, hd);
            WH_HIP(hipGetLastError());
        } else {
            WH_HIP(hipMemsetAsync(base, 0, s->kv_stream * sizeof(float), s->st));
        }
    }
    WH_HIP(hipStreamSynchronize(s->st));
    s->h_len[i] = n;
    s->h_hist[i].assign(tokens, tokens + n);
    return WH_OK;
}

// The persistent kernel serves a step of a one-stream sequence past position 0
// (at position 0 the step writes the cache row that the same step attends).
static bool mega_eligible(const wh_seq *s, const int32_t *active) {
    // the persistent kernel implements the reference mask only (attention mode 0)
    return s->mega_ok && s->S == 1 && s->m->attn_mode == 0 && (!active || active[0]) && s->h_len[0] >= 2 &&
           s->h_len[0] - 1 < s->m->n_ctx && s->h_len[0] + 1 <= s->hist_cap;
}

static int seq_forward_active(wh_seq *s, const int32_t *active) {
    int rc;
    if ((rc = upload_active(*s, active))) return rc;
    if ((rc = check_positions(*s))) return rc;
    return seq_forward(*s);
}

// One greedy step of the active streams with the sampling parameters already
// set per stream (set_sample_params).
static int step_greedy_impl(wh_seq *s, const int32_t *active, int32_t *out_ids, float *out_logits) {
    int rc;
    if (mega_eligible(s, active)) {
        int got = 0;
        if ((rc = mega_run(*s, 1, s->h_inv[0], s->h_supp[0], s->h_nst[0], s->hist_cap, -1, 0, out_logits, out_ids,
                           &got, nullptr, nullptr)))
            return rc;
        return WH_OK;
    }
    if ((rc = seq_forward_active(s, active))) return rc;
    const int V = s->m->n_vocab;
    {
        Prof p(*s, "sample", 0);
        if ((rc = launch_penalty_argmax(s->logits, s->hist, s->hist_len, s->hist_cap, s->active, s->S, V, s->m->eot,
                                        s->sb, s->st)))
            return rc;
        if ((rc = launch_argmax_final(s->sb, s->sb.cur, s->S, V, s->m->eot, s->active, s->hist, s->hist_len,
                                      s->hist_cap, s->tok, s->pos, s->out_ids, s->st)))
            return rc;
    }
    WH_HIP(hipMemcpyAsync(s->pinned_ids, s->out_ids, sizeof(int32_t) * s->S, hipMemcpyDeviceToHost, s->st));
    if (out_logits)
        WH_HIP(hipMemcpyAsync(out_logits, s->logits, sizeof(float) * (size_t)s->S * V, hipMemcpyDeviceToHost, s->st));
    WH_HIP(hipStreamSynchronize(s->st));
    if ((rc = batch_check(*s))) return rc;
    if (s->prof) s->prof_resolve();
    for (int i = 0; i < s->S; i++) {
        if (out_ids) out_ids[i] = s->h_active[i] ? s->pinned_ids[i] : -1;
        if (s->h_active[i]) {
            s->h_len[i]++;
            s->h_hist[i].push_back(s->pinned_ids[i]);
        }
    }
    return WH_OK;
}

int seq_step_greedy(wh_seq *s, const int32_t *active, float temperature, int32_t suppress_nst, float nst,
                    int32_t *out_ids, float *out_logits) {
    if (!s) return fail(WH_ERR_INVALID, "seq: null handle");
    WH_HIP(hipSetDevice(s->m->device));
    int rc;
    const float inv = temperature > 0 ? 1.0f / temperature : 1.0f;
    if ((rc = set_sample_params_all(*s, inv, suppress_nst, nst))) return rc;
    return step_greedy_impl(s, active, out_ids, out_logits);
}

// Up to n greedy steps of stream 0 with the reference's stop rules
// (decoder.go:441-485): EOT, more than 20 repeats of one token, max_len
// tokens. Returns the generated ids; the persistent kernel runs them on the
// device when it serves the sequence, else one multi-kernel step per token.
static int generate_impl(wh_seq *s, int32_t n, float temperature, int32_t suppress_nst, float nst, int32_t max_len,
                         int32_t *out_ids, int32_t *out_n, int &prev, int &streak) {
    *out_n = 0;
    if (s->h_len[0] == 0) return fail(WH_ERR_INVALID, "model: decode: forward: no tokens in state");
    WH_HIP(hipSetDevice(s->m->device));
    const float inv = temperature > 0 ? 1.0f / temperature : 1.0f;
    if (max_len > s->m->n_ctx) max_len = s->m->n_ctx;  // the reference caps at n_text_ctx
    int rc;
    int produced = 0;
    while (produced < n && s->h_len[0] < max_len) {
        int32_t id;
        if (mega_eligible(s, nullptr)) {
            int got = 0;
            if ((rc = mega_run(*s, n - produced, inv, suppress_nst, nst, max_len, prev, streak, nullptr,
                               out_ids ? out_ids + produced : nullptr, &got, &prev, &streak)))
                return rc;
            produced += got;
            *out_n = produced;
            const int32_t last = s->h_hist[0].back();
            if (got == 0 || last == s->m->eot || streak > 20) break;
            continue;
        }
        if ((rc = seq_step_greedy(s, nullptr, temperature, suppress_nst, nst, &id, nullptr))) return rc;
        if (out_ids) out_ids[produced] = id;
        produced++;
        *out_n = produced;
        if (id == s->m->eot) break;
        if (prev == id) streak++;
        else { streak = 1; prev = id; }
        if (streak > 20) break;
    }
    return WH_OK;
}

int seq_generate(wh_seq *s, int32_t n, float temperature, int32_t suppress_nst, float nst, int32_t max_len,
                 int32_t *out_ids, int32_t *out_n) {
    if (!s || !out_n) return fail(WH_ERR_INVALID, "seq: null argument");
    if (s->S != 1) return fail(WH_ERR_INVALID, "seq: generate needs a one-stream sequence");
    int prev = -1, streak = 0;
    return generate_impl(s, n, temperature, suppress_nst, nst, max_len, out_ids, out_n, prev, streak);
}

int seq_step_topk(wh_seq *s, const int32_t *active, int32_t k, float temperature, int32_t *out_tok, float *out_lp,
                  float *out_logits) {
    if (!s) return fail(WH_ERR_INVALID, "seq: null handle");
    if (k < 1 || k > 8) return fail(WH_ERR_INVALID, "seq: k must be in [1,8]");
    WH_HIP(hipSetDevice(s->m->device));
    int rc;
    if ((rc = seq_forward_active(s, active))) return rc;
    const float inv = temperature > 0 ? 1.0f / temperature : 1.0f;
    const int V = s->m->n_vocab;
    // the penalised copy `cur` is produced by the same pass that feeds greedy
    // selection; its argmax partials are unused here
    if ((rc = set_sample_params_all(*s, inv, 0, 0.0f))) return rc;
    if ((rc = launch_penalty_argmax(s->logits, s->hist, s->hist_len, s->hist_cap, s->active, s->S, V, s->m->eot,
                                    s->sb, s->st)))
        return rc;
    // one extra candidate exposes a tie at the k-th place
    const int kk = std::min(k + 1, 8);
    if ((rc = launch_topk(s->sb.cur, s->active, s->S, V, kk, inv, s->topk_tok, s->topk_lp, s->topk_logz, s->topk_part, s->st)))
        return rc;
    int32_t *h_tok = s->pinned_ids;
    float *h_lp = (float *)(s->pinned_ids + 16 * 8);
    float *h_logz = (float *)(s->pinned_ids + 2 * 16 * 8);
    WH_HIP(hipMemcpyAsync(h_tok, s->topk_tok, sizeof(int32_t) * s->S * kk, hipMemcpyDeviceToHost, s->st));
    WH_HIP(hipMemcpyAsync(h_lp, s->topk_lp, sizeof(float) * s->S * kk, hipMemcpyDeviceToHost, s->st));
    WH_HIP(hipMemcpyAsync(h_logz, s->topk_logz, sizeof(float) * s->S, hipMemcpyDeviceToHost, s->st));
    if (out_logits)
        WH_HIP(hipMemcpyAsync(out_logits, s->logits, sizeof(float) * (size_t)s->S * V, hipMemcpyDeviceToHost, s->st));
    WH_HIP(hipStreamSynchronize(s->st));
    if ((rc = batch_check(*s))) return rc;
    if (s->prof) s->prof_resolve();
    std::vector<float> row;
    for (int i = 0; i < s->S; i++) {
        const int32_t *t = h_tok + (size_t)i * kk;
        const float *l = h_lp + (size_t)i * kk;
        bool tie = false;
        for (int j = 0; j + 1 < kk; j++) tie |= (l[j] == l[j + 1]);
        if (s->h_active[i] && tie) {
            // Equal values at or inside the k-th place: the kept set and its
            // order depend on the reference's streaming replace-min scan
            // (decoder.go:1089-1121) followed by a stable sort of <= 12 items
            // (sort.Slice falls back to insertion sort there), so rerun that
            // scan exactly over the penalised row.
            row.resize(V);
            WH_HIP(hipMemcpy(row.data(), s->sb.cur + (size_t)i * V, sizeof(float) * V, hipMemcpyDeviceToHost));
            std::vector<int32_t> bt;
            std::vector<float> bv;
            int minpos = -1;
            float minval = 0.0f;
            for (int x = 0; x < V; x++) {
                const float sc = row[x] * inv;
                if ((int)bt.size() < k) {
                    bt.push_back(x);
                    bv.push_back(sc);
                    if (minpos < 0 || sc < minval) { minpos = (int)bt.size() - 1; minval = sc; }
                    continue;
                }
                if (sc <= minval) continue;
                bt[minpos] = x;
                bv[minpos] = sc;
                minpos = 0;
                minval = bv[0];
                for (int j = 1; j < (int)bv.size(); j++)
                    if (bv[j] < minval) { minval = bv[j]; minpos = j; }
            }
            std::vector<int> order(bt.size());
            for (size_t j = 0; j < order.size(); j++) order[j] = (int)j;
            for (size_t j = 0; j < bv.size(); j++) bv[j] -= h_logz[i];
            std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return bv[a] > bv[b]; });
            for (int j = 0; j < k; j++) {
                out_tok[(size_t)i * k + j] = j < (int)order.size() ? bt[order[j]] : -1;
                out_lp[(size_t)i * k + j] = j < (int)order.size() ? bv[order[j]] : 0.0f;
            }
            continue;
        }
        for (int j = 0; j < k; j++) {
            out_tok[(size_t)i * k + j] = s->h_active[i] ? t[j] : -1;
            out_lp[(size_t)i * k + j] = s->h_active[i] ? l[j] : 0.0f;
        }
    }
    return WH_OK;
}

void seq_destroy(wh_seq *s) { delete s; }

int seq_set_profiling(wh_seq *s, int32_t enable) {
    if (!s) return fail(WH_ERR_INVALID, "seq: null handle");
    WH_HIP(hipStreamSynchronize(s->st));
    s->pending.clear();
    s->ev_next = 0;
    s->prof_cats.clear();
    s->prof = enable != 0;
    return WH_OK;
}

int seq_profile_get(wh_seq *s, int32_t i, char *name, int32_t cap, double *ms, int64_t *launches, double *bytes) {
    if (!s) return fail(WH_ERR_INVALID, "seq: null handle");
    if (i < 0 || i >= (int32_t)s->prof_cats.size()) return fail(WH_ERR_INVALID, "seq: profile index out of range");
    const auto &c = s->prof_cats[i];
    if (name && cap > 0) {
        std::strncpy(name, c.name.c_str(), (size_t)cap - 1);
        name[cap - 1] = 0;
    }
    if (ms) *ms = c.ms;
    if (launches) *launches = c.launches;
    if (bytes) *bytes = c.bytes;
    return WH_OK;
}

int seq_persistent(wh_seq *s, int32_t *out, int64_t *launches) {
    if (!s || !out) return fail(WH_ERR_INVALID, "seq: null argument");
    *out = s->mega_ok && s->m->attn_mode == 0;
    if (launches) *launches = s->mega_launches;
    return WH_OK;
}

int seq_profile_count(wh_seq *s, int32_t *n) {
    if (!s || !n) return fail(WH_ERR_INVALID, "seq: null argument");
    *n = (int32_t)s->prof_cats.size();
    return WH_OK;
}

// ---- whole decode loops --------------------------------------------------------
namespace {

int cap_max_tokens(const wh_model &m, const wh_decode_params &p) {  // decoder.go:420-430
    int mt = p.max_tokens;
    if (mt <= 0) mt = m.n_ctx;
    if (m.n_ctx - p.prompt_len < mt) mt = m.n_ctx - p.prompt_len;
    return std::max(mt, 0);
}

int check_params(const wh_model &m, const wh_decode_params *p) {
    if (!p) return fail(WH_ERR_INVALID, "model: decode: null params");
    if (p->prompt_len < 0 || (p->prompt_len > 0 && !p->prompt)) return fail(WH_ERR_INVALID, "model: decode: invalid prompt");
    const float base = p->temperature == 0 ? 1.0f : p->temperature;
    if (p->logprob_thold > 0 && !p->no_fallback && base > 0)
        return fail(WH_ERR_UNSUPPORTED,
                    "model: decode: top-p fallback (LogprobThold > 0 without NoFallback) is non-deterministic in the "
                    "reference and is not supported");
    return WH_OK;
}

bool cancelled(const volatile int32_t *c) { return c && *c != 0; }

}  // namespace

// decoder.go:413-525 for n_streams independent streams (no vocabulary: no
// compression-ratio retries).
// Forward steps of the calling thread's last decode (wh_last_decode_steps).
thread_local int32_t g_decode_steps = 0;
int32_t last_decode_steps() { return g_decode_steps; }

int decode_greedy_batch(const wh_model *m, int32_t S, const float *const *encs, int32_t enc_len, int32_t enc_dim,
                        const wh_decode_params *params, int32_t *out_tokens, int32_t cap, int32_t *out_lens,
                        const volatile int32_t *cancel, int32_t dev) {
    int rc;
    g_decode_steps = 0;
    for (int i = 0; i < S; i++) {
        if ((rc = check_params(*m, &params[i]))) return rc;
        if (params[i].beam_size > 1)
            return fail(WH_ERR_UNSUPPORTED, "model: decode: the stream batch decodes greedily; stream " +
                                                std::to_string(i) + " asks for beam size " +
                                                std::to_string(params[i].beam_size));
    }
    wh_seq *sp = nullptr;
    if ((rc = seq_create(m, S, encs, enc_len, enc_dim, 0, &sp, dev))) return rc;
    std::unique_ptr<wh_seq, void (*)(wh_seq *)> s(sp, seq_destroy);
    std::vector<std::vector<int32_t>> toks(S);
    std::vector<int32_t> active(S, 1), maxt(S), streak(S, 0), prev(S, -1), ids(S);
    for (int i = 0; i < S; i++) {
        const wh_decode_params &p = params[i];
        toks[i].assign(p.prompt, p.prompt + p.prompt_len);
        maxt[i] = cap_max_tokens(*m, p);
        if ((rc = seq_set_tokens(s.get(), i, p.prompt, p.prompt_len, 0))) return rc;
        if ((int)toks[i].size() >= p.prompt_len + maxt[i]) active[i] = 0;
        else if (p.prompt_len == 0) return fail(WH_ERR_INVALID, "model: decode: forward: no tokens in state");
    }
    // each stream samples with its own temperature (0 => 1.0, decoder.go:416-419),
    // SuppressNST and NoSpeechThold
    std::vector<float> inv(S), nst(S);
    std::vector<int32_t> supp(S);
    for (int i = 0; i < S; i++) {
        const float base = params[i].temperature == 0 ? 1.0f : params[i].temperature;
        inv[i] = base > 0 ? 1.0f / base : 1.0f;
        supp[i] = params[i].suppress_nst;
        nst[i] = params[i].no_speech_thold;
    }
    if ((rc = set_sample_params(*s, inv.data(), supp.data(), nst.data()))) return rc;
    const wh_decode_params &p0 = params[0];
    const float base = p0.temperature == 0 ? 1.0f : p0.temperature;
    if (S == 1 && active[0]) {
        // the token loop runs on the device in chunks; cancellation is polled between chunks
        constexpr int CHUNK = 32;
        const int max_len = p0.prompt_len + maxt[0];
        std::vector<int32_t> got(CHUNK);
        int pv = -1, st = 0;
        while (active[0]) {
            if (cancelled(cancel)) return fail(WH_ERR_CANCELLED, "model: decode: cancelled: context canceled");
            int32_t n = 0;
            if ((rc = generate_impl(s.get(), CHUNK, base, p0.suppress_nst, p0.no_speech_thold, max_len, got.data(), &n,
                                    pv, st)))
                return fail(rc, std::string("model: decode: forward: ") + wh_last_error());
            toks[0].insert(toks[0].end(), got.begin(), got.begin() + n);
            g_decode_steps += n;
            if (n < CHUNK || toks[0].back() == m->eot || st > 20 || (int)toks[0].size() >= max_len) active[0] = 0;
        }
    }
    while (std::any_of(active.begin(), active.end(), [](int32_t a) { return a != 0; })) {
        if (cancelled(cancel)) return fail(WH_ERR_CANCELLED, "model: decode: cancelled: context canceled");
        if ((rc = step_greedy_impl(s.get(), active.data(), ids.data(), nullptr)))
            return fail(rc, std::string("model: decode: forward: ") + wh_last_error());
        g_decode_steps++;
        for (int i = 0; i < S; i++) {
            if (!active[i]) continue;
            const int32_t next = ids[i];
            toks[i].push_back(next);
            if (next == m->eot) { active[i] = 0; continue; }
            if (prev[i] == next) streak[i]++;
            else { streak[i] = 1; prev[i] = next; }
            if (streak[i] > 20) { active[i] = 0; continue; }
            if ((int)toks[i].size() >= params[i].prompt_len + maxt[i]) active[i] = 0;
        }
    }
    for (int i = 0; i < S; i++) {
        if ((int)toks[i].size() > cap) return fail(WH_ERR_INVALID, "model: decode: output capacity too small");
        std::memcpy(out_tokens + (size_t)i * cap, toks[i].data(), toks[i].size() * sizeof(int32_t));
        out_lens[i] = (int32_t)toks[i].size();
    }
    return WH_OK;
}

// decoder.go:528-726. The beam_size hypotheses run as one batch of beam
// objects (streams); every hypothesis is reset before its forward (P9), the cross
// K/V are shared and computed once (the reference recomputes identical values
// each step). The bookkeeping runs on the device: top-k with log-normaliser
// (launch_topk, plus the reference's scan for rows with ties), candidate ranking
// in Go's sort.Slice order, and the prune with the reference's in-place reuse of
// the beam objects (k_beam_select). The host reads the stop words once per step.
// Beam steps queued between two reads of the stop flags.
constexpr int BEAM_SYNC = 4;

int decode_beam(const wh_model *m, const float *enc, int32_t enc_len, int32_t enc_dim, const wh_decode_params *p,
                int32_t *out_tokens, int32_t cap, int32_t *out_len, const volatile int32_t *cancel, int32_t dev) {
    if (!p) return fail(WH_ERR_INVALID, "model: decode: null params");
    if (p->prompt_len < 0 || (p->prompt_len > 0 && !p->prompt)) return fail(WH_ERR_INVALID, "model: decode: invalid prompt");
    int rc;
    g_decode_steps = 0;
    const float temp = p->temperature == 0 ? 1.0f : p->temperature;
    const float inv = temp > 0 ? 1.0f / temp : 1.0f;
    const int bs = p->beam_size <= 0 ? 1 : p->beam_size;
    if (bs > 16)
        return fail(WH_ERR_UNSUPPORTED, "model: decode: beam size " + std::to_string(bs) +
                                            " exceeds the 16 hypotheses one batch holds");
    const int mt = cap_max_tokens(*m, *p);
    const int P = p->prompt_len;
    const int eot = m->eot;
    // the forward embeds the last token (decoder.go:757-759); the penalty skips ids out of range
    if (P > 0 && (p->prompt[P - 1] < 0 || p->prompt[P - 1] >= m->n_vocab) && mt > 0)
        return fail(WH_ERR_INVALID, "model: decode: beam search forward: model: decode: forward: invalid token ID " +
                                        std::to_string(p->prompt[P - 1]));
    if (mt <= 0 || (P > 0 && p->prompt[P - 1] == eot)) {
        // no step runs, or every hypothesis is finished from the start: the first is the prompt
        if (P > cap) return fail(WH_ERR_INVALID, "model: decode: output capacity too small");
        if (P > 0) std::memcpy(out_tokens, p->prompt, sizeof(int32_t) * P);
        *out_len = P;
        return WH_OK;
    }
    if (P == 0) return fail(WH_ERR_INVALID, "model: decode: beam search forward: model: decode: forward: no tokens in state");
    std::vector<const float *> encs(bs, enc);
    wh_seq *sp = nullptr;
    if ((rc = seq_create(m, bs, encs.data(), enc_len, enc_dim, 1, &sp, dev))) return rc;
    std::unique_ptr<wh_seq, void (*)(wh_seq *)> s(sp, seq_destroy);
    wh_seq &q = *s;
    // a slot's history grows by at most one token per earlier slot of its step
    const int hc = P + bs * (mt + 1) + 2, V = m->n_vocab, K = 5, KK = K + 1;
    int32_t *hist = nullptr, *gcap = nullptr, *order = nullptr, *nbeams = nullptr, *stop = nullptr;
    float *score = nullptr, *powtab = nullptr;
    if ((rc = q.alloc(&hist, (size_t)bs * hc)) || (rc = q.alloc(&gcap, (size_t)bs)) ||
        (rc = q.alloc(&order, (size_t)bs)) || (rc = q.alloc(&nbeams, 1)) || (rc = q.alloc(&stop, 4)) ||
        (rc = q.alloc(&score, (size_t)bs)) || (rc = q.alloc(&powtab, (size_t)hc + 2)))
        return rc;
    q.hist = hist;
    q.hist_cap = hc;
    WH_HIP(hipSetDevice(m->device));
    {
        // every beam object starts as the prompt (capacity P) with score 0; len^0.6 as the reference computes it
        std::vector<float> pw((size_t)hc + 2);
        for (size_t n = 0; n < pw.size(); n++) pw[n] = (float)std::pow((double)n, 0.6);
        std::vector<int32_t> h((size_t)bs * hc, 0), len(bs, P), tk(bs, p->prompt[P - 1]), ps(bs, P - 1), act(bs, 1),
            ord(bs);
        for (int b = 0; b < bs; b++) {
            std::memcpy(&h[(size_t)b * hc], p->prompt, sizeof(int32_t) * P);
            ord[b] = b;
        }
        const std::vector<float> sc(bs, 0.0f);
        const int32_t nb0 = bs, st0[4] = {0, -1, 0, 0};
        WH_HIP(hipMemcpy(powtab, pw.data(), sizeof(float) * pw.size(), hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(q.hist, h.data(), sizeof(int32_t) * h.size(), hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(q.hist_len, len.data(), sizeof(int32_t) * bs, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(gcap, len.data(), sizeof(int32_t) * bs, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(order, ord.data(), sizeof(int32_t) * bs, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(q.tok, tk.data(), sizeof(int32_t) * bs, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(q.pos, ps.data(), sizeof(int32_t) * bs, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(q.active, act.data(), sizeof(int32_t) * bs, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(score, sc.data(), sizeof(float) * bs, hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(nbeams, &nb0, sizeof(int32_t), hipMemcpyHostToDevice));
        WH_HIP(hipMemcpy(stop, st0, sizeof(st0), hipMemcpyHostToDevice));
        for (int b = 0; b < bs; b++) q.h_active[b] = 1;  // host mirror: the profiler's byte counts only
    }
    if ((rc = set_sample_params_all(q, inv, 0, 0.0f))) return rc;
    const int H = m->n_head, hd = m->n_state / H;
    for (int step = 0; step < mt; step++) {
        if (cancelled(cancel)) return fail(WH_ERR_CANCELLED, "model: decode: beam search cancelled: context canceled");
        // reset every hypothesis before its forward (P9): under the reference mask only cache row 0 is read
        if (m->attn_mode == 0) {
            const int count = bs * m->n_layer * 2 * H;
            hipLaunchKernelGGL(k_zero_rows, dim3(std::min(count, 1024)), dim3(64), 0, q.st, q.kv,
                               (size_t)m->n_ctx * hd, count, hd);
        } else {
            WH_HIP(hipMemsetAsync(q.kv, 0, q.kv_stream * sizeof(float) * bs, q.st));
        }
        WH_HIP(hipGetLastError());
        if ((rc = seq_forward(q)) ||
            (rc = launch_penalty_argmax(q.logits, q.hist, q.hist_len, hc, q.active, bs, V, eot, q.sb, q.st)) ||
            (rc = launch_topk(q.sb.cur, q.active, bs, V, KK, inv, q.topk_tok, q.topk_lp, q.topk_logz, q.topk_part, q.st)) ||
            (rc = launch_topk_ties(q.sb.cur, q.active, bs, V, K, KK, inv, q.topk_logz, q.topk_tok, q.topk_lp, q.st)) ||
            (rc = launch_beam_select(q.topk_tok, q.topk_lp, K, KK, q.hist, q.hist_len, gcap, hc, score, order, nbeams,
                                     q.active, q.tok, q.pos, stop, powtab, bs, eot, m->n_ctx, step, q.st)))
            return fail(rc, std::string("model: decode: beam search forward: ") + wh_last_error());
        // The flags are read every BEAM_SYNC steps and after the last: a step after
        // the one that set them leaves the beams as they are (k_beam_select), and
        // stop[3] names that step, so the outcome is the one of a check per step.
        if ((step + 1) % BEAM_SYNC != 0 && step + 1 < mt) continue;
        WH_HIP(hipMemcpyAsync(q.pinned_ids, stop, sizeof(int32_t) * 4, hipMemcpyDeviceToHost, q.st));
        WH_HIP(hipStreamSynchronize(q.st));
        if ((rc = batch_check(q))) return fail(rc, std::string("model: decode: beam search forward: ") + wh_last_error());
        if (q.prof) q.prof_resolve();
        const bool flagged = q.pinned_ids[0] || q.pinned_ids[1] >= 0;
        const int at = flagged ? q.pinned_ids[3] : step;  // the step that set the flags
        g_decode_steps = at + 1;
        if (q.pinned_ids[2]) return fail(WH_ERR_HIP, "model: decode: beam search: candidate sort stack exhausted");
        if (q.pinned_ids[0]) break;
        if (q.pinned_ids[1] >= 0 && at + 1 < mt)
            return fail(WH_ERR_INVALID, "model: decode: beam search forward: model: decode: forward: position " +
                                            std::to_string(q.pinned_ids[1]) + " >= context length " +
                                            std::to_string(m->n_ctx));
        if (q.pinned_ids[1] >= 0) break;
    }
    int32_t o0 = 0, len0 = 0;
    WH_HIP(hipMemcpy(&o0, order, sizeof(int32_t), hipMemcpyDeviceToHost));
    WH_HIP(hipMemcpy(&len0, q.hist_len + o0, sizeof(int32_t), hipMemcpyDeviceToHost));
    if (len0 > cap) return fail(WH_ERR_INVALID, "model: decode: output capacity too small");
    WH_HIP(hipMemcpy(out_tokens, q.hist + (size_t)o0 * hc, sizeof(int32_t) * len0, hipMemcpyDeviceToHost));
    *out_len = len0;
    return WH_OK;
}

}  // namespace wh
