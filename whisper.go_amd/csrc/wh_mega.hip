// Persistent decode kernel: whole greedy token steps of one stream in a single
// cooperative launch on gfx950 (internal/model/decoder.go:413-525 loop,
// :745-993 forward, reference-compatible attention mask).
//
// Under the reference mask the self-attention of a step past position 0
// attends KV row 0 only (internal/ml/attention.go:250-256), so its output
// sa_l = Wo_l . V0_l + ob_l does not depend on the step's activations, and the
// q,k,v rows the step adds to the cache are read by nobody within the step.
// Both are computed off the critical path by "side" workgroups while the
// cross-attention runs. One workgroup of 512 threads per CU walks these
// phases; each boundary is a data dependency between workgroups:
//   S  (once per step) embedding; side workgroups: sa_0 rows
//   B  item workgroups (one per (head, key chunk)): x1 = x_l + sa_l, LN2, q of
//      the head (64 rows of the cross query matrix), scores of the chunk and
//      its maximum. Side workgroups: LN1(x_l), q,k,v rows -> KV cache, and the
//      rows of sa_{l+1}.
//   C  item workgroups: head maximum, fast-exp weights, partial sum and P.V;
//      the last chunk of a head to finish combines the head
//   D  cross output rows: x2 = x1 + (Wo_c . attn + ob_c)
//   E  LN3 + fc1 rows + GELU
//   F  fc2 rows: x_{l+1} = x2 + (W2 . h + b2)
//   T  final LN + tied logits rows + repetition penalty + partial argmax;
//      every workgroup reduces the partials and takes the same next token.
// Each phase first issues the loads of everything it can (weight rows, LN
// parameters, biases, constant vectors) and then waits for its inputs.
//
// Cross-workgroup data moves through relaxed agent-scope atomic loads/stores
// (they bypass the non-coherent caches) and phase flags written after
// `s_waitcnt` has retired the data stores. Every wait is bounded: on timeout
// the error word is set, later waits return at once, the token loop stops and
// the host reports a failure.
//
// Addressing: the layer descriptors are copied into LDS once per launch; each
// phase reads the pointers it needs from there into scalar registers
// (readfirstlane) as global-address-space pointers, so weight loads are
// `global_load ... v_offset, s[base]` issued up front.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "wh_device.h"
#include "wh_internal.h"
#include "wh_mega.h"

namespace wh {
namespace mega {

constexpr int NT = THREADS;
constexpr int NW = WAVES;
constexpr int NC = NW;  // waves holding weight rows (all: more loads in flight beat a load-free poller)
constexpr int FS = FLAG_STRIDE;
constexpr unsigned SPIN_MAX = 1u << 22;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const uint8_t gu8;
typedef __attribute__((address_space(1))) const u32x4 gu4;
typedef __attribute__((address_space(1))) const uint16_t gu16;
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef __attribute__((address_space(1))) const float gf;
typedef __attribute__((address_space(1))) const f32x4 gf4;
typedef __attribute__((address_space(1))) float gfw;

__device__ __forceinline__ uint4 ld16(gu8 *p) {
    const u32x4 v = *(gu4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ld16f(gf *p) {
    const f32x4 v = *(gf4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ unsigned ld_u(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_f(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// threadIdx.x hidden from loop-invariant code motion. Every per-thread index
// and address below derives from it, so the compiler recomputes them inside
// each phase instead of hoisting them out of the token and layer loops, where
// the offsets of all phases would stay live at once and spill.
__device__ __forceinline__ int tid() {
    int t = (int)threadIdx.x;
    __asm__ volatile("" : "+v"(t));
    return t;
}

// A value that is the same on every lane, kept in a scalar register.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Index of this wave among the NC waves holding weight rows (-1: none).
__device__ __forceinline__ int cwave() { return uni(tid() >> 6) - (NW - NC); }

// A pointer that is the same on every lane, moved to scalar registers and
// typed as global memory.
template <typename G, typename T>
__device__ __forceinline__ G *glob(T *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (G *)(((uint64_t)hi << 32) | lo);
}

// A matrix as scalar global pointers to its planes (block counts come from d).
struct UView {
    gu8 *qs, *sc, *qh;
};
__device__ __forceinline__ UView uview(const MatView &m) {
    return UView{glob<gu8>(m.qs), glob<gu8>((const uint8_t *)m.sc), glob<gu8>((const uint8_t *)m.qh)};
}

// ---- cross-lane reductions: DPP within 16-lane rows, readlane across rows -------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// Sum over each 16-lane row (xor 1, xor 2, half-row mirror, row mirror); every
// lane of the row ends with the same value.
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Sum over the wave in a fixed order, (row0 + row1) + (row2 + row3); uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum16(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max16(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

#ifdef WH_MEGA_TRACE
// Diagnostic build only: thread 0 of every workgroup stamps the constant
// 100 MHz clock at each phase's start (point 0), after its wait (1) and before
// its publish (2), for the first TR_STEPS steps of a launch; points 3.. split
// a phase's work. Phase 6 is T, 7 the step-start phase S.
constexpr int TR_STEPS = 2, TR_MAXL = 33, TR_PTS = 8, TR_MAXW = 256;
__device__ long long g_trace[TR_STEPS * TR_MAXL * 8 * TR_PTS * TR_MAXW];
#define TRACE(step, l, ph, pt)                                                                                        \
    do {                                                                                                              \
        if ((step) < TR_STEPS && (l) < TR_MAXL && blockIdx.x < TR_MAXW && tid() == 0)                                 \
            g_trace[((((step) * TR_MAXL + (l)) * 8 + (ph)) * TR_PTS + (pt)) * TR_MAXW + blockIdx.x] = wall_clock64(); \
    } while (0)
#else
#define TRACE(step, l, ph, pt) \
    do {                       \
    } while (0)
#endif

// Retire this workgroup's coherent stores, then publish phase g in flags[slot].
__device__ __forceinline__ void publish(unsigned *flags, int slot, unsigned g) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid() == 0) st_u(&flags[(unsigned)slot * FS], g);
}

// Wait until flags[(first + i) * FS] >= g for i < count (1 <= count <= 256).
// Wave 0 polls with two rounds of loads in flight (the older round is tested
// while the newer one travels); the other waves wait at the barrier. The loads
// are unconditional (lanes past count re-read the last flag, one request per
// wave): predicated loads let the compiler test each value inside its own
// branch, right behind its load, which serialises the round trips. Addresses
// are a scalar base plus 32-bit lane offsets to keep the loop's registers few.
__device__ __forceinline__ void wait_flags(const unsigned *flags, int first, int count, unsigned g, unsigned *err) {
    const int t = tid();
    if (t < 64) {
        typedef __attribute__((address_space(1))) const unsigned gcu;
        gcu *base = glob<gcu>(flags);
        gcu *perr = glob<gcu>(err);
        unsigned off[4], v0[4], v1[4];
#pragma unroll
        for (int k = 0; k < 4; k++) off[k] = (unsigned)(first + min(t + 64 * k, count - 1)) * FS;
#pragma unroll
        for (int k = 0; k < 4; k++) v0[k] = __hip_atomic_load(base + off[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        unsigned e0 = __hip_atomic_load(perr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (unsigned spins = 0;; spins++) {
#pragma unroll
            for (int k = 0; k < 4; k++)
                v1[k] = __hip_atomic_load(base + off[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned e1 = __hip_atomic_load(perr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned lo = min(min(v0[0], v0[1]), min(v0[2], v0[3]));
            if (__all(lo >= g)) break;
            if (e0 != 0 || spins > SPIN_MAX) {  // another workgroup gave up, or this wait expired
                if (t == 0) atomicOr(err, 1u);
                break;
            }
#pragma unroll
            for (int k = 0; k < 4; k++) v0[k] = v1[k];
            e0 = e1;
        }
    }
    __syncthreads();
}

// LDS vectors keep each 32-element block in 36 slots: a lane reading its whole
// block then hits 4 banks no other lane of its 16-lane group uses.
__device__ __forceinline__ int pad(int i) { return i + ((i >> 5) << 2); }

// n floats (n even, src 8-byte aligned) of a coherent exchange vector into a
// padded LDS vector, two per 64-bit load.
__device__ __forceinline__ void xload_pad(float *dst, const float *src, int n) {
    for (int i = tid(); i < n / 2; i += NT) {
        const uint64_t v = __hip_atomic_load((const uint64_t *)src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *(float2 *)&dst[pad(2 * i)] = make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
    }
}
// same into a plain LDS vector
__device__ __forceinline__ void xload(float *dst, const float *src, int n) {
    for (int i = tid(); i < n / 2; i += NT) {
        const uint64_t v = __hip_atomic_load((const uint64_t *)src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *(float2 *)&dst[2 * i] = make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
    }
}

// ---- weight rows prefetched into registers ----------------------------------------
// Rows [r0, r1) of a workgroup; wave v takes rows r0+v, r0+v+NW, ...; lane l
// takes blocks l, l+64, ... of each row (PASSES passes). Slot s holds row
// k = s / PASSES of this wave and pass p = s % PASSES.
template <int TYPE, int MAXS>
struct Pre {
    uint4 a[MAXS];
    uint4 b[MAXS];  // second 16 bytes of a Q8_0 block
    uint32_t s[MAXS];
    uint32_t h[MAXS];
};

// Byte offsets stay 32-bit (the host checks every plane is below 4 GiB).
template <int TYPE>
__device__ __forceinline__ void load_blk(const UView &m, unsigned blk, uint4 &a, uint4 &b, uint32_t &s, uint32_t &h) {
    if constexpr (TYPE == 8) {
        a = ld16(m.qs + blk * 32u);
        b = ld16(m.qs + blk * 32u + 16u);
        s = *(gu16 *)(m.sc + blk * 2u);
    } else {
        a = ld16(m.qs + blk * 16u);
        if constexpr (TYPE == 3 || TYPE == 7) s = *(gu32 *)(m.sc + blk * 4u);
        else s = *(gu16 *)(m.sc + blk * 2u);
        if constexpr (TYPE == 6 || TYPE == 7) h = *(gu32 *)(m.qh + blk * 4u);
    }
}

// Loads are unconditional: a slot past the range re-reads the last valid row
// or block (row 0 for an empty range; a cache hit) and the dot products drop
// it, so no slot is ever undefined (undefined slots become loop-carried live
// ranges and spill) and no branch surrounds the loads.
template <int TYPE, int MAXS, int PASSES>
__device__ __forceinline__ void prefetch(Pre<TYPE, MAXS> &P, const UView &m, int nb, int r0, int r1) {
    const int lane = tid() & 63, cw = cwave();
    if (cw < 0) {
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            P.a[s] = make_uint4(0u, 0u, 0u, 0u);
            P.b[s] = make_uint4(0u, 0u, 0u, 0u);
            P.s[s] = 0u;
            P.h[s] = 0u;
        }
        return;
    }
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
        const int r = max(min(r0 + cw + NC * (s / PASSES), r1 - 1), 0);
        const int b = min(lane + 64 * (s % PASSES), nb - 1);
        load_blk<TYPE>(m, (unsigned)r * (unsigned)nb + (unsigned)b, P.a[s], P.b[s], P.s[s], P.h[s]);
    }
}

// f16 scale to f32 by the hardware conversion (exact for every finite value).
__device__ __forceinline__ float hf(uint32_t bits) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits); }

// dot of one prefetched block with 32 activations in registers
template <int TYPE>
__device__ __forceinline__ float block_dot(const uint4 &a, const uint4 &b, uint32_t s, uint32_t h, const float *x) {
    float acc = 0.0f;
    if constexpr (TYPE == 8) {
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int v = (int)w[t];
            acc += (float)((v << 24) >> 24) * x[4 * t] + (float)((v << 16) >> 24) * x[4 * t + 1] +
                   (float)((v << 8) >> 24) * x[4 * t + 2] + (float)(v >> 24) * x[4 * t + 3];
        }
        return hf(s) * acc;
    } else {
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
        const float off = (TYPE == 2) ? 8.0f : (TYPE == 6 ? 16.0f : 0.0f);
        float sx = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t byte = (w[t] >> (8 * k)) & 0xFFu;
                uint32_t lo = byte & 0xFu, hi = byte >> 4;
                const int e0 = 8 * t + 2 * k;
                if constexpr (TYPE == 6 || TYPE == 7) {
                    lo |= ((h >> e0) & 1u) << 4;
                    hi |= ((h >> (e0 + 1)) & 1u) << 4;
                }
                acc += ((float)lo - off) * x[e0] + ((float)hi - off) * x[e0 + 1];
                if constexpr (TYPE == 3 || TYPE == 7) sx += x[e0] + x[e0 + 1];
            }
        }
        if constexpr (TYPE == 3 || TYPE == 7) return hf(s & 0xFFFFu) * acc + hf(s >> 16) * sx;
        else return hf(s) * acc;
    }
}

// Activation block b of a padded LDS vector (16-byte aligned) into registers.
__device__ __forceinline__ void lds_block(const float *xs, int b, float (&xr)[32]) {
    const float4 *x4 = (const float4 *)(xs + b * 36);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float4 v = x4[j];
        xr[4 * j] = v.x;
        xr[4 * j + 1] = v.y;
        xr[4 * j + 2] = v.z;
        xr[4 * j + 3] = v.w;
    }
}

// Row dots of the prefetched slots: out[k] (same on every lane) is the dot of
// row r0 + cw + NC*k (cw = cwave()) with the padded LDS vector xs of nb
// blocks. Lanes past the last block and rows past r1 compute on duplicate
// data and add zero; the poller wave returns zeros.
template <int TYPE, int MAXS, int PASSES>
__device__ __forceinline__ void row_dots(const Pre<TYPE, MAXS> &P, int nb, int r0, int r1, const float *xs,
                                         float (&out)[MAXS / PASSES]) {
    const int lane = tid() & 63, cw = cwave();
    constexpr int K = MAXS / PASSES;
#pragma unroll
    for (int k = 0; k < K; k++) out[k] = 0.0f;
    if (cw < 0) return;
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int b = lane + 64 * p;
        float xr[32];
        lds_block(xs, min(b, nb - 1), xr);
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int s = k * PASSES + p;
            const int r = r0 + cw + NC * k;
            const float v = block_dot<TYPE>(P.a[s], P.b[s], P.s[s], P.h[s], xr);
            out[k] += (r < r1 && b < nb) ? v : 0.0f;
            __builtin_amdgcn_sched_barrier(0);  // decode one block at a time: bounded register use
        }
    }
#pragma unroll
    for (int k = 0; k < K; k++) out[k] = wave_sum(out[k]);
}

// out[lane] for lane < K (the row a lane finishes in an epilogue). out[] is
// wave-uniform, so each value is written into its lane with v_writelane; a
// select chain on the lane index is turned into a private (scratch) array.
template <int K>
__device__ __forceinline__ float pick(const float (&out)[K], int) {
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int s = uni(__builtin_bit_cast(int, out[k]));
        __asm__ volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(s), "i"(k));
    }
    return v;
}

// Per-lane bias of row r0 + cw + NC*lane (lane < K), clamped into [r0, r1);
// the poller wave loads nothing.
template <int K>
__device__ __forceinline__ float lane_bias(gf *bias, int r0, int r1) {
    const int lane = tid() & 63, cw = cwave();
    if (cw < 0) return 0.0f;
    return bias[max(min(r0 + cw + NC * min(lane, K - 1), r1 - 1), 0)];
}

// Row finished by this lane in an epilogue (lane < K of a compute wave), or -1.
template <int K>
__device__ __forceinline__ int lane_row(int r0, int r1) {
    const int lane = tid() & 63, cw = cwave();
    const int r = r0 + cw + NC * lane;
    return (cw >= 0 && lane < K && r < r1) ? r : -1;
}

// LayerNorm parameters of this thread's elements t, t+NT, t+2NT (n <= 3*NT).
struct LnPar {
    float w[3], b[3];
};
__device__ __forceinline__ void ln_load(LnPar &p, gf *w, gf *b, int n) {
    const int t = tid();
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int i = min(t + NT * j, n - 1);
        p.w[j] = w[i];
        p.b[j] = b[i];
    }
}

// LayerNorm (internal/ml/ops.go:153-202) of padded LDS xs[0..n) into padded
// LDS xo: mean, then the mean of squared deviations, sqrt in float64.
__device__ __forceinline__ void layernorm(const float *xs, float *xo, int n, const LnPar &p, float *red) {
    const int t = tid(), lane = t & 63, wave = t >> 6;
    float x[3];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int i = t + NT * j;
        x[j] = i < n ? xs[pad(i)] : 0.0f;
        s += x[j];
    }
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; i++) tot += red[i];
    const float mean = tot / (float)n;
    float v = 0.0f;
#pragma unroll
    for (int j = 0; j < 3; j++) {
        if (t + NT * j < n) {
            const float u = x[j] - mean;
            v += u * u;
        }
    }
    v = wave_sum(v);
    if (lane == 0) red[NW + wave] = v;
    __syncthreads();
    float tv = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; i++) tv += red[NW + i];
    const float var = tv / (float)n;
    const float sd = (float)sqrt((double)(var + 1e-5f));
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int i = t + NT * j;
        if (i < n) xo[pad(i)] = p.w[j] * (x[j] - mean) / sd + p.b[j];
    }
    __syncthreads();
}

__device__ __forceinline__ void better(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

// Logits rows of one chunk (<= NC*TS rows) with penalty and running argmax.
// pen[r - rv0] is the window count of row r.
template <int TYPE>
__device__ __forceinline__ void logits_chunk(const MegaArgs &a, const Pre<TYPE, TS> &P, int nb, int base, int end,
                                             const float *xn, const int *pen, int rv0, float &bv, int &bi,
                                             float &bv2, int &bi2) {
    const int lane = tid() & 63, cw = cwave();
    float out[TS];
    row_dots<TYPE, TS, 1>(P, nb, base, end, xn, out);
    if (cw < 0) return;
#pragma unroll
    for (int k = 0; k < TS; k++) {
        const int r = base + cw + NC * k;
        if (r < end) {
            float v = out[k];
            if (a.out_logits && lane == 0) a.out_logits[r] = v;
            const int cnt = pen[r - rv0];
            if (cnt > 0) v -= 2.0f * (float)cnt;
            const float s = v * a.inv_temp;
            better(s, r, bv, bi);
            if (r != a.eot) better(s, r, bv2, bi2);
            if (r == a.eot && lane == 0) st_f(a.eot_logit, v);
        }
    }
}

// LDS layout (floats): layer descriptors, then the vectors of k_decode.
__host__ __device__ inline int layer_floats(int L) { return (int)((L * sizeof(MegaLayer) + 15) / 16 * 4); }
__host__ __device__ inline int pen_floats(int V, int W) { return ((V + W - 1) / W + 3) / 4 * 4; }

// Side work of layer l (decoder.go:780-790 under the reference mask): LN1 of
// x_l (padded LDS xs) -> q,k,v rows [q0,q1), k and v stored in the KV cache at
// pos; rows [o0,o1) of sa_{l+1} = Wo_{l+1} . V0_{l+1} + ob_{l+1} (V0 in v0)
// into the exchange buffer. side_prefetch issues the loads.
template <int TYPE>
struct Side {
    Pre<TYPE, SQ> pq;
    Pre<TYPE, SO> po;
    LnPar p1;
    float qb, ob;  // per-lane biases of the epilogue rows
};

template <int TYPE>
__device__ __forceinline__ void side_prefetch(Side<TYPE> &S, const MegaArgs &a, const MegaLayer *ls, int l, int q0,
                                              int q1, int o0, int o1, int nbd, float *v0) {
    const MegaLayer &Ly = ls[l];
    prefetch<TYPE, SQ, 1>(S.pq, uview(Ly.sqkv), nbd, q0, q1);
    ln_load(S.p1, glob<gf>(Ly.ln1w), glob<gf>(Ly.ln1b), a.d);
    // v rows take the v bias; k rows have none; q rows are not used
    const int lane = tid() & 63, cw = max(cwave(), 0);
    const int r = max(min(q0 + cw + NC * min(lane, SQ - 1), q1 - 1), 0);
    S.qb = glob<gf>(Ly.svb)[max(r - 2 * a.d, 0)];
    // the last layer has no next layer: its own rows are loaded and not used
    const MegaLayer &Ln = ls[min(l + 1, a.L - 1)];
    prefetch<TYPE, SO, 1>(S.po, uview(Ln.so), nbd, o0, o1);
    S.ob = lane_bias<SO>(glob<gf>(Ln.sob), o0, o1);
    gf *kv = glob<gf>(Ln.kv) + (size_t)a.H * a.ctx * 64;  // V plane, row 0 of each head
    for (int i = tid(); i < a.d; i += NT) v0[pad(i)] = kv[(size_t)(i / 64) * a.ctx * 64 + (i % 64)];
}

template <int TYPE>
__device__ __forceinline__ void side_compute(const Side<TYPE> &S, const MegaArgs &a, const MegaLayer *ls, int l,
                                             int q0, int q1, int o0, int o1, int nbd, int pos, const float *xs,
                                             float *xn, const float *v0, float *red) {
    const int lane = tid() & 63;
    const int d = a.d;
    {
        layernorm(xs, xn, d, S.p1, red);
        float out[SQ];
        row_dots<TYPE, SQ, 1>(S.pq, nbd, q0, q1, xn, out);
        const float v = pick<SQ>(out, lane);
        const int r = lane_row<SQ>(q0, q1);
        // rows [0,d) q (unused under the reference mask), [d,2d) k, [2d,3d) v
        if (r >= d) {
            const int j = r % d, hh = j / 64, c = j % 64;
            const bool isv = r >= 2 * d;  // S.qb holds this lane's v bias then
            gfw *kv = glob<gfw>(ls[l].kv);
            kv[(isv ? (size_t)a.H * a.ctx * 64 : 0) + (size_t)hh * a.ctx * 64 + (size_t)pos * 64 + c] =
                isv ? v + S.qb : v;
        }
    }
    {
        __syncthreads();  // v0 complete
        float out[SO];
        row_dots<TYPE, SO, 1>(S.po, nbd, o0, o1, v0, out);
        const float v = pick<SO>(out, lane);
        const int r = lane_row<SO>(o0, o1);
        if (r >= 0 && l + 1 < a.L) st_f(&a.sa[(size_t)((l + 1) & 1) * d + r], v + S.ob);
    }
}

// Stage K rows [t0, t1) of head ih (a [enc_len][64] block of crossK) into LDS
// kst in the same layout with direct global->LDS loads (1 KiB per wave
// instruction), issued by waves 1.. only: wave 0 polls flags and its vector
// memory counter must stay free of long loads.
__device__ __forceinline__ void stage_k(const float *crossK, int enc_len, int ih, int t0, int t1, float *kst) {
    const int wave = uni(tid() >> 6), lane = tid() & 63;
    if (wave == 0) return;
    const float *src = crossK + ((size_t)ih * enc_len + t0) * 64;
    const int nvec = (t1 - t0) * 16;  // 16-byte vectors
    const int nblk = (nvec + 63) / 64;
    for (int b = wave - 1; b < nblk; b += NW - 1) {
        const int v = b * 64 + lane;
        if (v < nvec)
            __builtin_amdgcn_global_load_lds((void __attribute__((address_space(1))) *)(src + 4 * v),
                                             (void __attribute__((address_space(3))) *)(kst + b * 256), 16, 0, 0);
    }
}

template <int TYPE>
__global__ __launch_bounds__(NT, 1) void k_decode(MegaArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int d = a.d, H = a.H, L = a.L, W = gridDim.x, w = blockIdx.x;
    const int nbd = d / 32, nbf = 4 * d / 32;  // d is a multiple of 64
    const int d36 = nbd * 36;
    MegaLayer *ls = (MegaLayer *)lds;     // [L] layer descriptors
    float *xs = lds + layer_floats(L);    // [d36] x_l, later x2 (padded)
    float *x1s = xs + d36;                // [d36] x1 = x_l + sa_l (item), or V0 of the next layer (side)
    float *v0 = x1s;
    float *xn = x1s + d36;                // [4 d36] normalised / staged vectors (padded)
    float *sav = xn + 4 * d36;            // [d] sa_l (plain)
    float *xl_own = sav + d;              // [64] own rows of x_l
    float *x2_own = xl_own + 64;          // [64] own rows of x2
    float *red = x2_own + 64;             // [64]
    float *qh = red + 64;                 // [64] q of this workgroup's head
    float *sc = qh + 64;                  // [32*PKV] scores of this workgroup's chunk
    int *pen = (int *)(sc + 32 * PKV);    // [pen_floats] window counts of this workgroup's vocabulary rows
    float *kst = (float *)pen + pen_floats(a.V, gridDim.x);  // [chunk_len * 64] K rows of this item's chunk
    __shared__ unsigned last_flag;

    {
        const uint32_t *src = (const uint32_t *)a.layers;
        uint32_t *dst = (uint32_t *)ls;
        const int nw = L * (int)(sizeof(MegaLayer) / 4);
        for (int i = tid(); i < nw; i += NT) dst[i] = src[i];
        __syncthreads();
    }
    const Role &rl = a.roles[w];
    const int item = uni(rl.item), q0 = uni(rl.q0), q1 = uni(rl.q1), o0 = uni(rl.o0), o1 = uni(rl.o1);
    const bool has_item = item >= 0;
    const bool has_side = q1 > q0 || o1 > o0;
    const int ih = has_item ? item / a.C : 0, ic = has_item ? item % a.C : 0;
    const int t0 = ic * a.chunk_len, t1 = min(t0 + a.chunk_len, a.enc_len);
    // this item's share of its head's cross-query rows
    const int cq0 = ih * 64 + ic * 64 / a.C, cq1 = ih * 64 + (ic + 1) * 64 / a.C;
    const int rd0 = (int)((long)w * d / W), rd1 = (int)((long)(w + 1) * d / W);
    const int rf0 = (int)((long)w * 4 * d / W), rf1 = (int)((long)(w + 1) * 4 * d / W);
    const int rv0 = (int)((long)w * a.V / W), rv1 = (int)((long)(w + 1) * a.V / W);
    unsigned *iflags = a.flags + (size_t)W * FS;  // [H*C] item flags after the workgroup flags

    unsigned g = a.g0;
    int tok = a.tok0, len = a.len0, prev = a.prev0, streak = a.streak0;
    int produced = 0;

    for (int step = 0; step < a.n_steps; step++) {
        const int pos = len - 1;
        // ---------------- S: embedding, sa_0 rows ----------------
        {
            TRACE(step, 0, 7, 0);
            const int lane = tid() & 63, wave = tid() >> 6;
            Pre<TYPE, SO> po;
            prefetch<TYPE, SO, 1>(po, uview(ls[0].so), nbd, o0, o1);
            const float ob = lane_bias<SO>(glob<gf>(ls[0].sob), o0, o1);
            {
                gf *kv = glob<gf>(ls[0].kv) + (size_t)H * a.ctx * 64;
                for (int i = tid(); i < d; i += NT) v0[pad(i)] = kv[(size_t)(i / 64) * a.ctx * 64 + (i % 64)];
            }
            // token + positional embedding (decoder.go:756-773; quantised rows dequantised bit-exactly)
            for (int i = tid(); i < d; i += NT)
                xs[pad(i)] = dequant_elem<TYPE>(a.tok, tok, i >> 5, i & 31) + a.pos_emb[(size_t)pos * d + i];
            __syncthreads();
            for (int i = rd0 + tid(); i < rd1; i += NT) xl_own[i - rd0] = xs[pad(i)];
            {
                float out[SO];
                row_dots<TYPE, SO, 1>(po, nbd, o0, o1, v0, out);
                const float v = pick<SO>(out, lane);
                const int r = lane_row<SO>(o0, o1);
                if (r >= 0) st_f(&a.sa[r], v + ob);
            }
            TRACE(step, 0, 7, 2);
            publish(a.flags, w, ++g);
            if (has_item) stage_k(ls[0].crossK, a.enc_len, ih, t0, t1, kst);
        }
        for (int l = 0; l < L; l++) {
            const unsigned gin = g;  // x_l complete when every workgroup flag reaches gin
            // ---------------- B1: cross q rows (items) / side rows ----------------
            {
                const int lane = tid() & 63;
                TRACE(step, l, 1, 0);
                const MegaLayer &Ly = ls[l];
                if (has_item) {
                    Pre<TYPE, SCQ> pc;
                    LnPar p2;
                    prefetch<TYPE, SCQ, 1>(pc, uview(Ly.cq), nbd, cq0, cq1);
                    ln_load(p2, glob<gf>(Ly.ln2w), glob<gf>(Ly.ln2b), d);
                    const float qb = lane_bias<SCQ>(glob<gf>(Ly.cqb), cq0, cq1);
                    wait_flags(a.flags, 0, W, gin, a.err);
                    TRACE(step, l, 1, 1);
                    if (l > 0) xload_pad(xs, a.xg, d);
                    else xload(sav, a.sa, d);
                    __syncthreads();
                    for (int i = tid(); i < d; i += NT) x1s[pad(i)] = xs[pad(i)] + sav[i];
                    __syncthreads();
                    TRACE(step, l, 1, 3);
                    layernorm(x1s, xn, d, p2, red);
                    TRACE(step, l, 1, 4);
                    float out[SCQ];
                    row_dots<TYPE, SCQ, 1>(pc, nbd, cq0, cq1, xn, out);
                    const int r = lane_row<SCQ>(cq0, cq1);
                    if (r >= 0) st_f(&a.qx[r], pick<SCQ>(out, lane) + qb);
                    TRACE(step, l, 1, 2);
                    publish(iflags, item, ++g);
                } else {
                    Side<TYPE> S;
                    side_prefetch<TYPE>(S, a, ls, l, q0, q1, o0, o1, nbd, v0);
                    wait_flags(a.flags, 0, W, gin, a.err);
                    TRACE(step, l, 1, 1);
                    if (l > 0) xload_pad(xs, a.xg, d);
                    else xload(sav, a.sa, d);  // for D's x1 rows
                    __syncthreads();
                    side_compute<TYPE>(S, a, ls, l, q0, q1, o0, o1, nbd, pos, xs, xn, v0, red);
                    TRACE(step, l, 1, 2);
                    ++g;
                }
            }
            const unsigned gB1 = g;
            // ---------------- B2: scores of the chunk against the head's q ----------------
            ++g;
            const unsigned gB = g;
            if (has_item) {
                const int lane = tid() & 63, wave = tid() >> 6;
                TRACE(step, l, 0, 0);
                wait_flags(iflags, ih * a.C, a.C, gB1, a.err);
                TRACE(step, l, 0, 1);
                if (tid() < 32) {
                    const uint64_t v = __hip_atomic_load((const uint64_t *)(a.qx + ih * 64) + tid(), __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                    *(float2 *)&qh[2 * tid()] =
                        make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
                }
                __syncthreads();
                const float4 q4 = ((const float4 *)qh)[tid() & 15];
                const float4 *k4 = (const float4 *)kst;
                float mx = -INFINITY;
#pragma unroll
                for (int j = 0; j < PKV; j++) {
                    const int tu = t0 + (j * NT + tid()) / 16;
                    // keys past the chunk re-read its last staged key; the scores drop them
                    const int t = min(tu, t1 - 1);
                    const float4 kr = k4[(t - t0) * 16 + (tid() & 15)];
                    const float part = row_sum16(q4.x * kr.x + q4.y * kr.y + q4.z * kr.z + q4.w * kr.w);
                    if (tu < t1) {
                        const float s = part * a.scale;
                        if ((tid() & 15) == 0) sc[tu - t0] = s;
                        mx = fmaxf(mx, s);
                    }
                }
                mx = wave_max(mx);
                if (lane == 0) red[wave] = mx;
                __syncthreads();
                if (tid() == 0) {
                    float m = red[0];
                    for (int i = 1; i < NW; i++) m = fmaxf(m, red[i]);
                    st_f(&a.cmax[item], m);
                }
                TRACE(step, l, 0, 2);
                publish(iflags, item, gB);
            }
            // ---------------- C: softmax weights, partial P.V, head combine ----------------
            ++g;
            const unsigned gC = g;
            if (has_item) {
                const int lane = tid() & 63, wave = tid() >> 6;
                TRACE(step, l, 2, 0);
                const MegaLayer &Ly = ls[l];
                float4 vr[PKV];
                gf *Vv = glob<gf>(Ly.crossV) + (size_t)ih * a.enc_len * 64;
                const int tt = tid();
#pragma unroll
                for (int j = 0; j < PKV; j++) {
                    const int t = min(t0 + (j * NT + tt) / 16, t1 - 1);
                    vr[j] = ld16f(Vv + (unsigned)t * 64u + 4u * (unsigned)(tt & 15));
                }
                wait_flags(iflags, ih * a.C, a.C, gB, a.err);
                TRACE(step, l, 2, 1);
                // chunk maxima of the head: all loads in flight before the first use
                float cm[CMAX];
#pragma unroll
                for (int i = 0; i < CMAX; i++) cm[i] = i < a.C ? ld_f(&a.cmax[ih * a.C + i]) : -INFINITY;
                float M = cm[0];
#pragma unroll
                for (int i = 1; i < CMAX; i++) M = fmaxf(M, cm[i]);
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
                float es = 0.0f;
#pragma unroll
                for (int j = 0; j < PKV; j++) {
                    const int t = t0 + (j * NT + tid()) / 16;
                    if (t < t1) {
                        const float e = fast_exp(sc[t - t0] - M);
                        acc.x += e * vr[j].x; acc.y += e * vr[j].y; acc.z += e * vr[j].z; acc.w += e * vr[j].w;
                        if ((tid() & 15) == 0) es += e;
                    }
                }
#pragma unroll
                for (int o = 16; o < 64; o <<= 1) {
                    acc.x += __shfl_xor(acc.x, o, 64);
                    acc.y += __shfl_xor(acc.y, o, 64);
                    acc.z += __shfl_xor(acc.z, o, 64);
                    acc.w += __shfl_xor(acc.w, o, 64);
                }
                es = wave_sum(es);
                float4 *red4 = (float4 *)xn;  // [NW][16]
                if (lane < 16) red4[wave * 16 + lane] = acc;
                if (lane == 0) red[wave] = es;
                __syncthreads();
                float *pv = a.parts + (size_t)item * 65;
                if (tid() < 16) {
                    float4 r = red4[tid()];
                    for (int v2 = 1; v2 < NW; v2++) {
                        const float4 t4 = red4[v2 * 16 + tid()];
                        r.x += t4.x; r.y += t4.y; r.z += t4.z; r.w += t4.w;
                    }
                    st_f(&pv[4 * tid()], r.x);
                    st_f(&pv[4 * tid() + 1], r.y);
                    st_f(&pv[4 * tid() + 2], r.z);
                    st_f(&pv[4 * tid() + 3], r.w);
                }
                if (tid() == 0) {
                    float s = 0.0f;
                    for (int v2 = 0; v2 < NW; v2++) s += red[v2];
                    st_f(&pv[64], s);
                }
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                // the last chunk of this head to arrive combines the head
                if (tid() == 0) {
                    const unsigned old = __hip_atomic_fetch_add(&a.hcount[(size_t)(l * H + ih) * FS], 1u,
                                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    last_flag = ((old + 1) % (unsigned)a.C) == 0;
                }
                __syncthreads();
                if (last_flag && tid() < 64) {
                    float ps[CMAX], po[CMAX];
#pragma unroll
                    for (int i = 0; i < CMAX; i++) {
                        const float *p2 = a.parts + (size_t)(ih * a.C + min(i, a.C - 1)) * 65;
                        ps[i] = i < a.C ? ld_f(&p2[64]) : 0.0f;
                        po[i] = i < a.C ? ld_f(&p2[tid()]) : 0.0f;
                    }
                    float sum = 0.0f, o = 0.0f;
#pragma unroll
                    for (int i = 0; i < CMAX; i++) {
                        sum += ps[i];
                        o += po[i];
                    }
                    st_f(&a.attn[ih * 64 + tid()], o * (1.0f / sum));
                    __builtin_amdgcn_s_waitcnt(0);
                    if (tid() == 0) st_u(&a.hflags[(size_t)ih * FS], gC);
                }
                TRACE(step, l, 2, 2);
                if (has_side) {
                    // fewer side workgroups than the side rows need: items take a share after C
                    __syncthreads();
                    Side<TYPE> S;
                    side_prefetch<TYPE>(S, a, ls, l, q0, q1, o0, o1, nbd, v0);
                    __syncthreads();
                    side_compute<TYPE>(S, a, ls, l, q0, q1, o0, o1, nbd, pos, xs, xn, v0, red);
                }
            }
            // ---------------- D: cross out rows -> x2 ----------------
            {
                const int lane = tid() & 63, wave = tid() >> 6;
                TRACE(step, l, 3, 0);
                const MegaLayer &Ly = ls[l];
                Pre<TYPE, SD> pd;
                prefetch<TYPE, SD, 1>(pd, uview(Ly.co), nbd, rd0, rd1);
                const float cb = lane_bias<SD>(glob<gf>(Ly.cob), rd0, rd1);
                wait_flags(a.hflags, 0, H, gC, a.err);
                TRACE(step, l, 3, 1);
                xload_pad(xn, a.attn, d);
                __syncthreads();
                {
                    float out[SD];
                    row_dots<TYPE, SD, 1>(pd, nbd, rd0, rd1, xn, out);
                    const float v = pick<SD>(out, lane);
                    const int r = lane_row<SD>(rd0, rd1);
                    if (r >= 0) {
                        const float x1 = xl_own[r - rd0] + sav[r];
                        const float x2 = x1 + (v + cb);
                        x2_own[r - rd0] = x2;
                        st_f(&a.x2[r], x2);
                    }
                }
                TRACE(step, l, 3, 2);
                publish(a.flags, w, ++g);
            }
            const unsigned gD = g;
            // ---------------- E: LN3 + fc1 + GELU ----------------
            {
                const int lane = tid() & 63, wave = tid() >> 6;
                TRACE(step, l, 4, 0);
                const MegaLayer &Ly = ls[l];
                Pre<TYPE, SE> pe;
                LnPar p3;
                prefetch<TYPE, SE, 1>(pe, uview(Ly.fc1), nbd, rf0, rf1);
                const float fb = lane_bias<SE>(glob<gf>(Ly.fc1b), rf0, rf1);
                ln_load(p3, glob<gf>(Ly.ln3w), glob<gf>(Ly.ln3b), d);
                wait_flags(a.flags, 0, W, gD, a.err);
                TRACE(step, l, 4, 1);
                xload_pad(xs, a.x2, d);
                __syncthreads();
                TRACE(step, l, 4, 3);
                layernorm(xs, xn, d, p3, red);
                TRACE(step, l, 4, 4);
                {
                    float out[SE];
                    row_dots<TYPE, SE, 1>(pe, nbd, rf0, rf1, xn, out);
                    TRACE(step, l, 4, 5);
                    const float v = pick<SE>(out, lane);
                    const int r = lane_row<SE>(rf0, rf1);
                    if (r >= 0) st_f(&a.hbuf[r], gelu_ref(v + fb));
                }
                TRACE(step, l, 4, 2);
                publish(a.flags, w, ++g);
            }
            const unsigned gE = g;
            // ---------------- F: fc2 rows -> x_{l+1} ----------------
            {
                const int lane = tid() & 63, wave = tid() >> 6;
                TRACE(step, l, 5, 0);
                const MegaLayer &Ly = ls[l];
                Pre<TYPE, SD * PFC2> pf;
                prefetch<TYPE, SD * PFC2, PFC2>(pf, uview(Ly.fc2), nbf, rd0, rd1);
                const float fb = lane_bias<SD>(glob<gf>(Ly.fc2b), rd0, rd1);
                // the next layer's K chunk (this layer's was consumed in B2)
                if (has_item && l + 1 < L) stage_k(ls[l + 1].crossK, a.enc_len, ih, t0, t1, kst);
                wait_flags(a.flags, 0, W, gE, a.err);
                TRACE(step, l, 5, 1);
                xload_pad(xn, a.hbuf, 4 * d);
                if (l + 1 < L) xload(sav, a.sa + (size_t)((l + 1) & 1) * d, d);
                __syncthreads();
                TRACE(step, l, 5, 3);
                {
                    float out[SD];
                    row_dots<TYPE, SD * PFC2, PFC2>(pf, nbf, rd0, rd1, xn, out);
                    TRACE(step, l, 5, 5);
                    const float v = pick<SD>(out, lane);
                    const int r = lane_row<SD>(rd0, rd1);
                    if (r >= 0) {
                        const float x = x2_own[r - rd0] + (v + fb);
                        xl_own[r - rd0] = x;
                        st_f(&a.xg[r], x);
                    }
                }
                TRACE(step, l, 5, 2);
                publish(a.flags, w, ++g);
            }
        }
        const unsigned gF = g;
        // ---------------- T: final LN, logits rows, penalty, argmax ----------------
        {
            const int lane = tid() & 63, wave = tid() >> 6;
            TRACE(step, L, 6, 0);
            const UView vt = uview(a.tok);
            Pre<TYPE, TS> p0, p1;
            const int CH = NC * TS;
            LnPar pf;
            prefetch<TYPE, TS, 1>(p0, vt, nbd, rv0, min(rv0 + CH, rv1));
            ln_load(pf, glob<gf>(a.lnw), glob<gf>(a.lnb), d);
            for (int i = tid(); i < rv1 - rv0; i += NT) pen[i] = 0;
            wait_flags(a.flags, 0, W, gF, a.err);
            TRACE(step, L, 6, 1);
            xload_pad(xs, a.xg, d);
            // repetition window (decoder.go:1000-1016): counts of this workgroup's rows
            const int start = len > 128 ? len - 128 : 0, nwin = len - start;
            if (tid() < nwin) {
                const int id = (int)ld_u((const unsigned *)&a.hist[start + tid()]);
                if (id >= rv0 && id < rv1) atomicAdd(&pen[id - rv0], 1);
            }
            __syncthreads();
            TRACE(step, L, 6, 3);
            layernorm(xs, xn, d, pf, red);
            TRACE(step, L, 6, 4);
            float bv = -INFINITY, bv2 = -INFINITY;
            int bi = 0x7FFFFFFF, bi2 = 0x7FFFFFFF;
            for (int base = rv0; base < rv1; base += 2 * CH) {
                const int b1 = base + CH;
                prefetch<TYPE, TS, 1>(p1, vt, nbd, min(b1, rv1 - 1), min(b1 + CH, rv1));
                logits_chunk<TYPE>(a, p0, nbd, base, min(base + CH, rv1), xn, pen, rv0, bv, bi, bv2, bi2);
                if (b1 < rv1) {
                    const int b2 = b1 + CH;
                    prefetch<TYPE, TS, 1>(p0, vt, nbd, min(b2, rv1 - 1), min(b2 + CH, rv1));
                    logits_chunk<TYPE>(a, p1, nbd, b1, min(b1 + CH, rv1), xn, pen, rv0, bv, bi, bv2, bi2);
                }
            }
            TRACE(step, L, 6, 5);
            float *rv = red;
            float *rv2 = red + NW;
            int *ri = (int *)(red + 2 * NW), *ri2 = (int *)(red + 3 * NW);
            if (lane == 0) { rv[wave] = bv; ri[wave] = bi; rv2[wave] = bv2; ri2[wave] = bi2; }
            __syncthreads();
            if (tid() == 0) {
                for (int i = 1; i < NW; i++) { better(rv[i], ri[i], rv[0], ri[0]); better(rv2[i], ri2[i], rv2[0], ri2[0]); }
                st_f(&a.pval[w], rv[0]);
                st_u((unsigned *)&a.pidx[w], (unsigned)ri[0]);
                st_f(&a.pval[W + w], rv2[0]);
                st_u((unsigned *)&a.pidx[W + w], (unsigned)ri2[0]);
            }
            TRACE(step, L, 6, 2);
            publish(a.flags, w, ++g);
            wait_flags(a.flags, 0, W, g, a.err);
            TRACE(step, L, 6, 6);
            // every workgroup reduces the partials the same way
            if (tid() < 64) {
                float b1 = -INFINITY, b2 = -INFINITY;
                int i1 = 0x7FFFFFFF, i2 = 0x7FFFFFFF;
                for (int i = tid(); i < W; i += 64) {
                    better(ld_f(&a.pval[i]), (int)ld_u((const unsigned *)&a.pidx[i]), b1, i1);
                    better(ld_f(&a.pval[W + i]), (int)ld_u((const unsigned *)&a.pidx[W + i]), b2, i2);
                }
                for (int o = 32; o > 0; o >>= 1) {
                    float ov = __shfl_xor(b1, o, 64);
                    int oi = __shfl_xor(i1, o, 64);
                    better(ov, oi, b1, i1);
                    ov = __shfl_xor(b2, o, 64);
                    oi = __shfl_xor(i2, o, 64);
                    better(ov, oi, b2, i2);
                }
                if (tid() == 0) {
                    int id = (i1 == 0x7FFFFFFF) ? 0 : i1;
                    if (a.suppress_nst && a.eot >= 0 && a.eot < a.V && id == a.eot && ld_f(a.eot_logit) < -a.nst)
                        id = (i2 == 0x7FFFFFFF) ? a.eot : i2;
                    red[63] = __int_as_float(id);
                }
            }
            __syncthreads();
            tok = __float_as_int(red[63]);
            __syncthreads();
        }
        // history append and the reference's stop rules (decoder.go:462-484)
        if (w == 0 && tid() == 0) {
            st_u((unsigned *)&a.hist[len], (unsigned)tok);
            a.out_tokens[produced] = tok;
        }
        len++;
        produced++;
        bool stop = (tok == a.eot) || (len >= a.max_len);
        if (prev == tok) streak++;
        else { streak = 1; prev = tok; }
        if (streak > 20) stop = true;
        if (stop || ld_u(a.err)) break;
    }
    if (w == 0 && tid() == 0) {
        a.state_out[0] = produced;
        a.state_out[1] = prev;
        a.state_out[2] = streak;
        a.state_out[3] = (int)g;
    }
}

#ifdef WH_MEGA_TRACE
extern "C" int wh_mega_trace_read(void *out, size_t bytes) {
    if (bytes > sizeof(g_trace)) bytes = sizeof(g_trace);
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_trace), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -2;
}
#endif

size_t lds_bytes(int d, int L, int V, int W, int chunk_len) {
    const int d36 = ((d + 31) / 32) * 36;
    return sizeof(float) *
           (size_t)(layer_floats(L) + 6 * d36 + d + 64 * 4 + 32 * PKV + pen_floats(V, W) + chunk_len * 64);
}

int launch_decode(uint32_t type, int grid, const MegaArgs &a, hipStream_t st) {
    void *args[] = {(void *)&a};
    const size_t shmem = lds_bytes(a.d, a.L, a.V, grid, a.chunk_len);
    const void *fn = nullptr;
    switch (type) {
    case 2: fn = (const void *)k_decode<2>; break;
    case 3: fn = (const void *)k_decode<3>; break;
    case 6: fn = (const void *)k_decode<6>; break;
    case 7: fn = (const void *)k_decode<7>; break;
    case 8: fn = (const void *)k_decode<8>; break;
    default: return fail(WH_ERR_UNSUPPORTED, "persistent decode: unsupported weight type");
    }
    WH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem));
    WH_HIP(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(NT), args, shmem, st));
    return WH_OK;
}

}  // namespace mega
}  // namespace wh
