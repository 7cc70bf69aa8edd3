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

// DPP exchange within rows of 16 lanes
template <int CTRL>
__device__ __forceinline__ float dpp16(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// max and sum over the 16 lanes of a row, left in every lane
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp16<0xB1>(v));
    v = fmaxf(v, dpp16<0x4E>(v));
    v = fmaxf(v, dpp16<0x141>(v));
    return fmaxf(v, dpp16<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp16<0xB1>(v);
    v += dpp16<0x4E>(v);
    v += dpp16<0x141>(v);
    return v + dpp16<0x140>(v);
}

constexpr int ATQ = 64;         // queries per workgroup
constexpr int ATK = 64;         // keys per tile
constexpr int ATS = ATQ + 4;    // LDS row stride (floats): 16-byte rows, rotated banks
constexpr size_t AT_LDS = 4 * 64 * ATS * sizeof(float);

// SDPA of one head, 64 queries per workgroup, head size 64
// (ml/attention.go:193-281 with the fast-exp softmax of attention.go:93-131):
// scores = (q . k) * scale; weight = fastexp(score - row max) / row sum;
// out = weights . V. Pass 1 finds every row's maximum over all keys; pass 2
// recomputes the scores tile by tile, forms the fast-exp weights against that
// maximum and accumulates weights . V and the row sums; the output is the
// accumulation times 1 / sum. Thread (qi, ki) holds queries 4qi..4qi+3 against
// keys (pass 1, scores) or output columns (pass 2, P.V) 4ki..4ki+3; the 16
// threads of a query group are one DPP row. Q, K, V, out are [T, d] with head
// h in columns 64h..64h+63.
__global__ __launch_bounds__(256) void k_enc_attn64(const float *Q, const float *K, const float *V, int T, int d,
                                                     float scale, float *out) {
    extern __shared__ float lds[];
    float(*Qt)[ATS] = (float(*)[ATS])lds;                  // [dim][query]
    float(*Kt)[ATS] = (float(*)[ATS])(lds + 64 * ATS);     // [dim][key]
    float(*Vs)[ATS] = (float(*)[ATS])(lds + 128 * ATS);    // [key][dim]
    float(*Pt)[ATS] = (float(*)[ATS])(lds + 192 * ATS);    // [key][query]
    const int h = blockIdx.y, q0 = blockIdx.x * ATQ, tid = threadIdx.x;
    const int qi = tid >> 4, ki = tid & 15;
    const size_t col = (size_t)h * 64;
    for (int i = tid; i < 64 * 64; i += 256) {
        const int t = i >> 6, c = i & 63;
        Qt[c][t] = q0 + t < T ? Q[(size_t)(q0 + t) * d + col + c] : 0.0f;
    }
    // scores of the thread's 4 x 4 block against the staged key tile
    const auto tile_scores = [&](float (&s)[4][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) s[i][j] = 0.0f;
#pragma unroll 8
        for (int c = 0; c < 64; c++) {
            const float4 qv = *(const float4 *)&Qt[c][4 * qi];
            const float4 kv = *(const float4 *)&Kt[c][4 * ki];
            const float qa[4] = {qv.x, qv.y, qv.z, qv.w}, ka[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) s[i][j] = __builtin_fmaf(qa[i], ka[j], s[i][j]);
        }
    };
    const auto stage_k = [&](int k0) __attribute__((always_inline)) {
        for (int i = tid; i < 64 * 64; i += 256) {
            const int t = i >> 6, c = i & 63;
            Kt[c][t] = k0 + t < T ? K[(size_t)(k0 + t) * d + col + c] : 0.0f;
        }
    };
    // pass 1: row maxima
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (int k0 = 0; k0 < T; k0 += ATK) {
        __syncthreads();
        stage_k(k0);
        __syncthreads();
        float s[4][4];
        tile_scores(s);
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (k0 + 4 * ki + j < T)
#pragma unroll
                for (int i = 0; i < 4; i++) mx[i] = fmaxf(mx[i], s[i][j] * scale);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) mx[i] = row16_max(mx[i]);
    // pass 2: fast-exp weights, P.V and row sums
    float acc[4][4], rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < T; k0 += ATK) {
        __syncthreads();
        stage_k(k0);
        for (int i = tid; i < 64 * 64; i += 256) {
            const int t = i >> 6, c = i & 63;
            Vs[t][c] = k0 + t < T ? V[(size_t)(k0 + t) * d + col + c] : 0.0f;
        }
        __syncthreads();
        float s[4][4];
        tile_scores(s);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool ok = k0 + 4 * ki + j < T;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = ok ? fast_exp(s[i][j] * scale - mx[i]) : 0.0f;
                rs[i] += e;
                Pt[4 * ki + j][4 * qi + i] = e;
            }
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < ATK; k++) {
            const float4 pv = *(const float4 *)&Pt[k][4 * qi];
            const float4 vv = *(const float4 *)&Vs[k][4 * ki];
            const float pa[4] = {pv.x, pv.y, pv.z, pv.w}, va[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(pa[i], va[j], acc[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float sum = row16_sum(rs[i]);
        const int t = q0 + 4 * qi + i;
        if (t >= T) continue;
        // the row maximum's own weight is fast_exp(0) = 1, so sum >= 1 (the
        // reference's uniform-weight branch for sum == 0 cannot be taken)
        const float inv = 1.0f / sum;
        float4 o = make_float4(acc[i][0] * inv, acc[i][1] * inv, acc[i][2] * inv, acc[i][3] * inv);
        *(float4 *)&out[(size_t)t * d + col + 4 * ki] = o;
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

int launch_enc_attn(const float *Q, const float *K, const float *V, int T, int d, int H, float *out, hipStream_t s) {
    const int hd = d / H;
    const float scale = (float)(1.0 / sqrt((double)hd));
    if (hd == 64 && d % 4 == 0) {
        WH_HIP(hipFuncSetAttribute((const void *)k_enc_attn64, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)AT_LDS));
        hipLaunchKernelGGL(k_enc_attn64, dim3((T + ATQ - 1) / ATQ, H), dim3(256), AT_LDS, s, Q, K, V, T, d, scale,
                           out);
    } else {
        hipLaunchKernelGGL(k_enc_attn_any, dim3(T, H), dim3(64), (size_t)T * sizeof(float), s, Q, K, V, T, d, hd,
                           scale, out);
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

}  // namespace wh
