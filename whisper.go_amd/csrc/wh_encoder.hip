// Encoder kernels (internal/model/encoder.go:265-396): the conv stem's im2col
// staging, GELU (+ positional embedding), and the full (unmasked) self-attention
// of every head over all frames. The projections run on k_cross_gemm (fp32
// matrix cores, quantised weights decoded bit-exactly), the LayerNorms on
// k_layernorm.
#include <hip/hip_runtime.h>

#include <cmath>

#include "wh_device.h"
#include "wh_internal.h"

namespace wh {

namespace {

// ml/conv.go:19-70 as a product: row t of the staged matrix holds the kernel
// window of output frame t, element ci * 3 + k = in(ci, t * stride - 1 + k)
// (zero outside [0, tin) and past 3 cin, up to the padded width K), so that
// conv(t, oc) = bias[oc] + sum_j E[t, j] W[oc, j] with W the [out_c, in_c, 3]
// weight flattened. in(ci, tt) sits at in[ci * sc + tt * st].
__global__ void k_im2col(const float *in, int64_t sc, int64_t st, int cin, int tin, int stride, int tout, int K,
                         float *out) {
    const int64_t n = (int64_t)tout * K;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(i / K), j = (int)(i % K);
        const int ci = j / 3, k = j - 3 * ci, it = t * stride - 1 + k;
        out[i] = (ci < cin && it >= 0 && it < tin) ? in[ci * sc + (int64_t)it * st] : 0.0f;
    }
}

// x = GELU(x) (+ pos, the same [rows, d] layout), ops.go:102-122 with tanh in float64.
__global__ void k_gelu_add(float *x, const float *pos, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float g = gelu_ref(x[i]);
        x[i] = pos ? g + pos[i] : g;
    }
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int AK = 64;       // keys per tile
constexpr int AKS = AK + 4;  // K tile row stride (floats): 16-byte rows, 16 rows cover the 64 banks once

// SDPA of one head with head size 64 on the fp32 matrix cores
// (ml/attention.go:193-281 with the fast-exp softmax of attention.go:93-131):
// scores = (q . k) * scale; weight = fastexp(score - row max) / row sum;
// out = weights . V. Each wave owns 32 queries and one of KS interleaved shares
// of the key tiles (64 keys each); the QW x KS waves of a workgroup stage KS
// tiles per round in LDS (the next round's loads in flight while the current one
// is used).
//
// The products are formed transposed, S^T = K Q^T and O^T = V^T P^T, with
// v_mfma_f32_32x32x2f32: its accumulator gives lane l the column l % 32 (one
// query) and rows 8 (i / 4) + 4 (l / 32) + i % 4 in register i (keys, or output
// dimensions). A query's row maximum and sum are then a lane's own values and
// its partner lane l ^ 32, and register i of the weights is exactly the B
// operand (key 8 (i / 4) + i % 4 from lanes 0-31, that key + 4 from lanes
// 32-63) of the P.V step that takes the V rows of those two keys as A.
// In S^T = K Q^T, MFMA k-index 0 carries dimensions 0-31 and index 1
// dimensions 32-63, so each lane keeps its query's half row of q in registers.
//
// Pass 1 finds every row's maximum of scale * score over all keys (the shares'
// maxima combined through LDS); pass 2 recomputes the scores, forms the fast-exp
// weights against that maximum, accumulates weights . V and the row sums; the
// shares' sums and products are added in share order and the output is the
// accumulation times 1 / sum. Keys past T weigh 0 (their V rows are staged as
// zeros), queries past T are not stored. Q, K, V, out are [T, d] with head h in
// columns 64h..64h+63.
template <int QW, int KS>
constexpr size_t attn_lds() {
    return sizeof(float) * ((size_t)KS * AK * (AKS + 64) + (size_t)KS * QW * 32);
}

template <int QW, int KS>
__global__ __launch_bounds__(64 * QW * KS) void k_enc_attn_mfma(const float *Q, const float *K, const float *V, int T,
                                                                int d, float scale, float *out) {
    constexpr int NT = 64 * QW * KS, NL = AK * 16 * KS / NT;  // float4 of a round's tiles per thread
    static_assert(AK * 16 * KS % NT == 0, "a round is whole float4 rounds of the workgroup");
    extern __shared__ float4 lds_f4[];  // attn_lds<QW, KS>() bytes
    float(*Ks)[AK][AKS] = (float(*)[AK][AKS])lds_f4;                       // [KS][AK][AKS]
    float(*Vs)[AK][64] = (float(*)[AK][64])((float *)lds_f4 + KS * AK * AKS);  // [KS][AK][64]
    float(*mxs)[QW][32] = (float(*)[QW][32])((float *)lds_f4 + KS * AK * (AKS + 64));
    const int h = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int qw = wave % QW, ks = wave / QW;
    const int ql = lane & 31, half = lane >> 5;
    const int q = blockIdx.x * 32 * QW + qw * 32 + ql;
    const size_t col = (size_t)h * 64;
    float qr[32];
    {
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 *src = (const float4 *)(Q + (size_t)q * d + col + 32 * half);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 v = q < T ? src[j] : z;
            qr[4 * j] = v.x; qr[4 * j + 1] = v.y; qr[4 * j + 2] = v.z; qr[4 * j + 3] = v.w;
        }
    }
    // round staging: float4 i of a round is tile i / 1024 of the round (keys
    // r0 + 64 (i / 1024) ..), key (i % 1024) / 16, dimensions 4 (i % 16) ..
    const auto load_round = [&](const float *src, int r0, float4 (&r)[NL]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NL; j++) {
            const int i = tid + j * NT, key = r0 + (i >> 4);
            r[j] = key < T ? *(const float4 *)(src + (size_t)key * d + col + 4 * (i & 15))
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    const auto store_k = [&](const float4 (&r)[NL]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NL; j++) {
            const int i = tid + j * NT;
            *(float4 *)&Ks[i >> 10][(i >> 4) & 63][4 * (i & 15)] = r[j];
        }
    };
    const auto store_v = [&](const float4 (&r)[NL]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NL; j++) {
            const int i = tid + j * NT;
            *(float4 *)&Vs[i >> 10][(i >> 4) & 63][4 * (i & 15)] = r[j];
        }
    };
    // S^T of this wave's staged tile: s0 keys 0-31, s1 keys 32-63, this lane's query
    const auto scores = [&](f32x16 &s0, f32x16 &s1) __attribute__((always_inline)) {
        s0 = f32x16{};
        s1 = f32x16{};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 ka = *(const float4 *)&Ks[ks][ql][32 * half + 4 * j];
            const float4 kb = *(const float4 *)&Ks[ks][32 + ql][32 * half + 4 * j];
            s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.x, qr[4 * j], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kb.x, qr[4 * j], s1, 0, 0, 0);
            s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.y, qr[4 * j + 1], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kb.y, qr[4 * j + 1], s1, 0, 0, 0);
            s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.z, qr[4 * j + 2], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kb.z, qr[4 * j + 2], s1, 0, 0, 0);
            s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.w, qr[4 * j + 3], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kb.w, qr[4 * j + 3], s1, 0, 0, 0);
        }
    };
    // key of register i within its 32-key half of the tile
    const auto rkey = [&](int i) __attribute__((always_inline)) { return 8 * (i >> 2) + 4 * half + (i & 3); };
    constexpr int RK = AK * KS;  // keys per round
    float4 kr[NL], vr[NL];
    // pass 1: row maxima
    float mx = -INFINITY;
    load_round(K, 0, kr);
    for (int r0 = 0; r0 < T; r0 += RK) {
        __syncthreads();
        store_k(kr);
        __syncthreads();
        if (r0 + RK < T) load_round(K, r0 + RK, kr);
        const int k0 = r0 + AK * ks;
        if (k0 < T) {
            f32x16 s0, s1;
            scores(s0, s1);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                if (k0 + rkey(i) < T) mx = fmaxf(mx, s0[i] * scale);
                if (k0 + 32 + rkey(i) < T) mx = fmaxf(mx, s1[i] * scale);
            }
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (KS > 1) {
        if (lane < 32) mxs[ks][qw][ql] = mx;
        __syncthreads();
        mx = mxs[0][qw][ql];
#pragma unroll
        for (int k = 1; k < KS; k++) mx = fmaxf(mx, mxs[k][qw][ql]);
    }
    // pass 2: fast-exp weights, P.V and row sums
    f32x16 o0 = {}, o1 = {};  // output dimensions 0-31 and 32-63
    float rs = 0.0f;
    load_round(K, 0, kr);
    load_round(V, 0, vr);
    for (int r0 = 0; r0 < T; r0 += RK) {
        __syncthreads();
        store_k(kr);
        store_v(vr);
        __syncthreads();
        if (r0 + RK < T) {
            load_round(K, r0 + RK, kr);
            load_round(V, r0 + RK, vr);
        }
        const int k0 = r0 + AK * ks;
        if (k0 < T) {
            f32x16 s0, s1;
            scores(s0, s1);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                s0[i] = k0 + rkey(i) < T ? fast_exp(s0[i] * scale - mx) : 0.0f;
                s1[i] = k0 + 32 + rkey(i) < T ? fast_exp(s1[i] * scale - mx) : 0.0f;
                rs += s0[i] + s1[i];
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float *va = Vs[ks][rkey(i)], *vb = Vs[ks][32 + rkey(i)];
                o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(va[ql], s0[i], o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(va[32 + ql], s0[i], o1, 0, 0, 0);
                o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[ql], s1[i], o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[32 + ql], s1[i], o1, 0, 0, 0);
            }
        }
    }
    rs += __shfl_xor(rs, 32, 64);
    if (KS > 1) {
        // shares 1.. post their sums and products over the K tiles; share 0 adds them in order
        float *post = &Ks[0][0][0];  // [KS - 1][QW][64 lanes][33]
        __syncthreads();
        if (ks > 0) {
            float *p = post + (((size_t)(ks - 1) * QW + qw) * 64 + lane) * 33;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                p[i] = o0[i];
                p[16 + i] = o1[i];
            }
            p[32] = rs;
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int k = 1; k < KS; k++) {
            const float *p = post + (((size_t)(k - 1) * QW + qw) * 64 + lane) * 33;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                o0[i] += p[i];
                o1[i] += p[16 + i];
            }
            rs += p[32];
        }
    }
    if (q >= T) return;
    // the row maximum's own weight is fast_exp(0) = 1, so rs >= 1 (the
    // reference's uniform-weight branch for a zero sum cannot be taken)
    const float inv = 1.0f / rs;
    float *dst = out + (size_t)q * d + col + 4 * half;
#pragma unroll
    for (int a = 0; a < 4; a++) {
        *(float4 *)(dst + 8 * a) = make_float4(o0[4 * a] * inv, o0[4 * a + 1] * inv, o0[4 * a + 2] * inv,
                                               o0[4 * a + 3] * inv);
        *(float4 *)(dst + 32 + 8 * a) = make_float4(o1[4 * a] * inv, o1[4 * a + 1] * inv, o1[4 * a + 2] * inv,
                                                    o1[4 * a + 3] * inv);
    }
}

// The same SDPA for any head size: one 64-thread workgroup per (query, head);
// the row's scores in LDS, then the reference's order of operations (scale,
// fast exp against the row maximum, weights = e * (1 / sum), weights . V).
__global__ __launch_bounds__(64) void k_enc_attn_any(const float *Q, const float *K, const float *V, int T, int d,
                                                     int hd, float scale, float *out) {
    extern __shared__ float sc[];
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const float *q = Q + (size_t)t * d + (size_t)h * hd;
    float mx = -INFINITY;
    for (int j = lane; j < T; j += 64) {
        const float *k = K + (size_t)j * d + (size_t)h * hd;
        float s = 0.0f;
        for (int c = 0; c < hd; c++) s = __builtin_fmaf(q[c], k[c], s);
        s *= scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sum = 0.0f;
    for (int j = lane; j < T; j += 64) {
        const float e = fast_exp(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    __syncthreads();
    const float inv = sum == 0.0f ? 0.0f : 1.0f / sum;
    const float uni = 1.0f / (float)T;
    for (int c = lane; c < hd; c += 64) {
        float o = 0.0f;
        for (int j = 0; j < T; j++) {
            const float w = sum == 0.0f ? uni : sc[j] * inv;
            o = __builtin_fmaf(w, V[(size_t)j * d + (size_t)h * hd + c], o);
        }
        out[(size_t)t * d + (size_t)h * hd + c] = o;
    }
}

int grid_for(int64_t n) { return (int)std::min<int64_t>((n + 255) / 256, 8192); }

}  // namespace

int launch_im2col(const float *in, int64_t sc, int64_t st, int cin, int tin, int stride, int tout, int K, float *out,
                  hipStream_t s) {
    hipLaunchKernelGGL(k_im2col, dim3(grid_for((int64_t)tout * K)), dim3(256), 0, s, in, sc, st, cin, tin, stride,
                       tout, K, out);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int launch_gelu_add(float *x, const float *pos, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_gelu_add, dim3(grid_for(n)), dim3(256), 0, s, x, pos, n);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// Loads this file's code object (the runtime does it on first use otherwise).
int warm_encoder_kernels() {
    hipFuncAttributes attr;
    WH_HIP(hipFuncGetAttributes(&attr, (const void *)k_enc_attn_mfma<4, 2>));
    return WH_OK;
}

int launch_enc_attn(const float *Q, const float *K, const float *V, int T, int d, int H, float *out, hipStream_t s) {
    const int hd = d / H;
    const float scale = (float)(1.0 / sqrt((double)hd));
    if (hd == 64 && d % 4 == 0 && ((uintptr_t)Q & 15) == 0 && ((uintptr_t)K & 15) == 0 &&
        ((uintptr_t)V & 15) == 0 && ((uintptr_t)out & 15) == 0) {
        constexpr int QW = 4, KS = 2;  // 4 x 32 queries per workgroup, keys in 2 shares
        constexpr size_t lds = attn_lds<QW, KS>();
        WH_HIP(hipFuncSetAttribute((const void *)k_enc_attn_mfma<QW, KS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)lds));
        hipLaunchKernelGGL((k_enc_attn_mfma<QW, KS>), dim3((T + 32 * QW - 1) / (32 * QW), H), dim3(64 * QW * KS), lds,
                           s, Q, K, V, T, d, scale, out);
    } else {
        hipLaunchKernelGGL(k_enc_attn_any, dim3(T, H), dim3(64), (size_t)T * sizeof(float), s, Q, K, V, T, d, hd,
                           scale, out);
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

}  // namespace wh
