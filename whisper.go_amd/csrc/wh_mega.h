// Persistent decode kernel: argument block shared by the host launcher and the
// gfx950 kernel (wh_mega.hip).
#pragma once

#include <cstddef>
#include <cstdint>

#include "wh_device.h"

namespace wh {
namespace mega {

struct MegaLayer {
    MatView sqkv, so, cq, co, fc1, fc2;  // sqkv: q, k, v rows stacked ([3d, d])
    const float *ln1w, *ln1b, *svb, *sob, *ln2w, *ln2b, *cqb, *cob, *ln3w, *ln3b, *fc1b, *fc2b;
    const float *crossK, *crossV;  // [enc_len][d] of this layer (stream 0)
    float *kv;                     // [2][H][n_ctx][64] of this layer (stream 0)
};

// Work of one workgroup. item >= 0: (head, key chunk) = (item / C, item % C)
// of the cross-attention; the side rows are the self-attention q,k,v rows
// [q0, q1) of the layer and the self-attention output rows [o0, o1) of the
// next layer, computed while the cross-attention runs.
struct Role {
    int32_t item;
    int32_t q0, q1, o0, o1;
    int32_t pad[3];
};

struct MegaArgs {
    const MegaLayer *layers;
    const Role *roles;  // [grid]
    int L, d, H, ctx, V, enc_len;
    int C, chunk_len;  // key chunks per head and keys per chunk
    float scale;       // float32(1/sqrt(64))
    MatView tok;
    const float *pos_emb, *lnw, *lnb;
    // token loop state
    int32_t *hist;  // history (prompt + generated), coherent accesses only
    int tok0, len0, prev0, streak0;
    int n_steps, max_len, eot, suppress_nst;
    float inv_temp, nst;
    int32_t *out_tokens;  // [n_steps]
    float *out_logits;    // raw logits of the last step, or null
    int32_t *state_out;   // produced, prev, streak, final phase index
    // exchange buffers
    float *xg, *sa, *x2, *hbuf, *attn, *cmax, *parts, *pval, *eot_logit, *qx;
    int32_t *pidx;
    unsigned *flags, *hflags, *hcount, *err;
    unsigned g0;
};

constexpr int THREADS = 512;
constexpr int WAVES = THREADS / 64;
constexpr int FLAG_STRIDE = 16;
constexpr int PKV = 8;      // float4 of K (and of V) per thread: 256-key chunks
constexpr int CMIN = 4;     // key chunks per head at least (so a chunk's q rows fit SCQ)
constexpr int CMAX = 8;     // key chunks per head at most (2048 encoder frames)
constexpr int PFC2 = 3;     // fc2 input passes: n_state <= 64*3*32/4 = 1536
// register slots (rows) per wave: a workgroup holds WAVES * slots rows of each kind
constexpr int SCQ = 2;      // cross query rows of one chunk: 64 / C <= 16 (C >= 4)
constexpr int SQ = 4;       // q,k,v side rows
constexpr int SO = 2;       // self-attention output side rows
constexpr int SD = 2;       // cross output rows (also fc2 rows)
constexpr int SE = 5;       // fc1 rows
constexpr int TS = 6;       // logits rows per chunk

// Dynamic LDS bytes of the kernel for n_state d, L layers, V vocabulary rows,
// a grid of W workgroups and chunk_len keys per chunk.
size_t lds_bytes(int d, int L, int V, int W, int chunk_len);

}  // namespace mega
}  // namespace wh
