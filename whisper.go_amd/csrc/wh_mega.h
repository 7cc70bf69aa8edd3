// Persistent decode kernel: argument block shared by the host launcher and the
// gfx950 kernel (wh_mega.hip).
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>

#include "wh_device.h"

namespace wh {
namespace mega {

struct MegaLayer {
    MatView sqkv, so, cq, co, fc1, fc2;  // sqkv: q, k, v rows stacked ([3d, d])
    const float *ln1w, *ln1b, *svb, *sob, *ln2w, *ln2b, *cqb, *cob, *ln3w, *ln3b, *fc1b, *fc2b;
    const float *cqc, *cqe, *f1c, *f1e;  // folded LN2 / LN3 row constants (see Layer)
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
    // Exchange buffers of 8-byte {float value (low word), phase (high word)}
    // pairs, each stored with one atomic 64-bit store: a reader polls the
    // pairs themselves until they carry the phase it waits for.
    uint64_t *xg;         // [d] x_l
    uint64_t *sa;         // [2][d] sa_l by layer parity
    uint64_t *x2;         // [d]
    uint64_t *hbuf;       // [4d] GELU(fc1)
    uint64_t *attn;       // [d] cross-attention output
    uint64_t *qx;         // [d] cross query
    uint64_t *cmax;       // [H*C] chunk score maxima
    uint64_t *parts;      // [H*C][65] chunk P.V sums and weight sums
    uint64_t *part;       // [W][4] argmax partials: value, index, value without EOT, index
    uint64_t *eot_logit;  // [1]
    unsigned *err;
    unsigned g0;
};

constexpr int THREADS = 512;
constexpr int WAVES = THREADS / 64;
constexpr int CWAVES = WAVES - 1;  // waves 1.. hold weight rows; wave 0 polls, exchanges and publishes
constexpr int PKQ = 2;      // scores: 128 keys per pass of 512 threads, 256 keys per chunk at most
constexpr int PVK = 10;     // P.V: float4 of V per compute thread, 448 * 10 / 16 = 280 keys at most
constexpr int CHUNK_MAX = 256;
constexpr int SC_FLOATS = (CHUNK_MAX + 31) / 32 * 32;  // LDS scores of a chunk
constexpr int CMIN = 5;     // key chunks per head at least
constexpr int CMAX = 8;     // key chunks per head at most (2048 encoder frames)
constexpr int XD = 21;      // exchange pairs per lane of a d-vector load: n_state <= 1344
constexpr int XH = 12;      // exchange pairs per compute lane of the 4d-vector load: 4d <= 7*64*12
constexpr int XS = 3;       // exchange pairs per compute lane of a d-vector load: d <= 7*64*3
constexpr int XP = 9;       // exchange pairs per lane of a head's chunk sums: CMAX * 65 <= 576
constexpr int XT = 16;      // exchange pairs per lane of the argmax partials: 4 * 256
// register slots (rows) per compute wave: a workgroup holds CWAVES * slots rows of each kind
constexpr int SQ = 5;       // q,k,v side rows
constexpr int SO = 2;       // self-attention output side rows
constexpr int SD = 1;       // cross output rows
constexpr int TS = 6;       // logits rows per chunk
// flat splits (blocks per compute lane, rows per compute wave): cross query rows
// of a chunk, fc1 rows, fc2 rows of a workgroup
constexpr int FQ = 1, RQ = 3;
constexpr int FE = 2, RE = 4;
constexpr int FF = 2, RF = 2;

// Whether the flat split of nrows rows of nb blocks over the compute waves fits
// P blocks per lane, RS rows per wave and three waves per row (the kernel's
// limits; rows are posted by communication lanes, so nrows <= 64).
inline bool flat_fits(int nrows, int nb, int P, int RS) {
    if (nrows < 0 || nrows > 64 || nb <= 0 || nb > 255) return false;
    const int n = nrows * nb;
    int cover[64] = {0};
    const int A = std::min(CWAVES, std::max(1, 2 * nrows));  // waves with items
    for (int c = 0; c < A; c++) {
        const int i0 = c * n / A, i1 = (c + 1) * n / A;
        if (i1 - i0 > 64 * P) return false;
        if (i1 <= i0) continue;
        const int ra = i0 / nb, rb = (i1 - 1) / nb;
        if (rb - ra + 1 > RS) return false;
        for (int r = ra; r <= rb; r++)
            if (++cover[r] > 3) return false;
    }
    return true;
}

// Dynamic LDS bytes of the kernel for n_state d, L layers, V vocabulary rows,
// a grid of W workgroups and chunk_len keys per chunk.
size_t lds_bytes(int d, int L, int V, int W, int chunk_len);

}  // namespace mega
}  // namespace wh
