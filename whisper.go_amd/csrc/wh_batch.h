// Persistent forward of a batch of decoder states (beam hypotheses or
// independent streams) in one cooperative launch per token step; shared by the
// host (wh_seq.cpp) and the kernel (wh_batch.hip). Not part of the C ABI.
#pragma once

#include <cstddef>
#include <cstdint>

#include "wh_device.h"

namespace wh {
namespace batch {

constexpr int NT = 512;              // threads per workgroup (8 waves, two per SIMD)
constexpr int SMAX = 16;             // streams per launch
constexpr int RW = 1;                // GEMV rows per lane group and pass
constexpr int XBUDGET = 112 * 1024;  // LDS bytes for staged activation matrices [S][cols]
constexpr int LNMAX = 2048;          // widest LayerNorm whose weights are staged in LDS
constexpr int CHUNK = 128;           // keys per cross-attention item
constexpr int CMAX = 8;              // key chunks per head at most

struct BLayer {
    MatView sqkv, so, cq, co, fc1, fc2;  // q,k,v stacked [3d, d]
    const float *ln1w, *ln1b, *svb, *sob, *ln2w, *ln2b, *cqb, *cob, *ln3w, *ln3b, *fc1b, *fc2b;
    float *kv;                            // this layer's KV cache of stream 0 ([2][H][ctx][64]); streams kv_stream apart
    const float *const *kbase;            // [S] cross K of this layer per stream ([H][enc_len][64])
    const float *const *vbase;
};

struct BArgs {
    const BLayer *layers;
    int L, d, H, ctx, V, enc_len, S;
    int xchunks;                          // key chunks per head in cross attention (S * H * xchunks <= grid)
    size_t kv_stream;                     // floats between two streams' KV caches
    MatView tok;                          // token embedding = tied logits matrix
    const float *pos_emb, *lnw, *lnb;
    const int32_t *tokv, *posv, *active;  // [S]
    // exchanged between workgroups as {tag, value} pairs (value in the low word):
    // activations [S][d] ([S][4d] for h), self-attention outputs [L][S][d], and
    // per key chunk of a head its P.V and weight sum [S][H][xchunks][65] and its
    // maximum score [S][H][xchunks]
    uint64_t *x, *x2, *q, *h, *attn, *sa, *pv, *xmax;
    float *logits;                        // [S][V]
    unsigned *flags;                      // [grid] last published phase
    unsigned *err;                        // set when a wait gives up
    float scale;                          // 1/sqrt(64)
    int mfma;                             // GEMV rows on the matrix cores
};

constexpr int LMAX = 32;              // layers at most

// Rows of a workgroup's GEMV pass: lane groups of g lanes (32 for widths up to
// 1024, else 64), 64 / g rows per group.
constexpr int pass_rows(int d) { return NT / 64 * RW * (d <= 1024 ? 2 : 1); }

// LDS bytes of the kernel: the staged matrix (32 floats per block), its block
// sums, LayerNorm weight and bias, per-state scalars, a reduction area and the
// layer descriptors.
constexpr size_t LDS_BYTES =
    (size_t)XBUDGET + (size_t)(XBUDGET / 128) * 4 + 2 * LNMAX * 4 + 256 + 4096 + LMAX * sizeof(BLayer);
static_assert(sizeof(BLayer) % 8 == 0, "layer descriptors are copied in 8-byte words");

}  // namespace batch
}  // namespace wh
