// Persistent forward of a batch of decoder states (beam hypotheses or
// independent streams) in one cooperative launch per token step; shared by the
// host (wh_seq.cpp) and the kernel (wh_batch.hip). Not part of the C ABI.
#pragma once

#include <cstddef>
#include <cstdint>

#include "wh_device.h"

namespace wh {
namespace batch {

constexpr int NT = 256;          // threads per workgroup (4 waves, one per SIMD)
constexpr int SMAX = 8;          // streams per launch
constexpr int XBUDGET = 128 * 1024;  // LDS bytes for the staged activation matrix [S][cols]

struct BLayer {
    MatView sqkv, so, cq, co, fc1, fc2;  // q,k,v stacked [3d, d]
    const float *ln1w, *ln1b, *svb, *sob, *ln2w, *ln2b, *cqb, *cob, *ln3w, *ln3b, *fc1b, *fc2b;
    float *kv;                            // this layer's KV cache of stream 0 ([2][H][ctx][64]); streams kv_stream apart
    const float *const *kbase;            // [S] cross K of this layer per stream ([enc_len, d], P3 view)
    const float *const *vbase;
};

struct BArgs {
    const BLayer *layers;
    int L, d, H, ctx, V, enc_len, S, chunks, chunk_len;
    size_t kv_stream;                     // floats between two streams' KV caches
    MatView tok;                          // token embedding = tied logits matrix
    const float *pos_emb, *lnw, *lnb;
    const int32_t *tokv, *posv, *active;  // [S]
    float *x, *x1, *x2, *q, *attn, *h, *logits;     // activations [S][d] ([S][4d] for h, [S][V] logits)
    float *scores, *cmax, *psum, *pv;               // cross-attention scratch [S][H][enc_len] / [S][H][chunks](x64)
    unsigned *flags;                      // [grid] barrier phases
    unsigned *err;                        // set when a wait gives up
    float scale;                          // 1/sqrt(64)
};

// LDS bytes of the kernel: the staged matrix (32 floats per block), its block
// sums, and a small reduction area.
constexpr size_t LDS_BYTES = (size_t)XBUDGET + (size_t)(XBUDGET / 128) * sizeof(float) + 4096;

}  // namespace batch
}  // namespace wh
