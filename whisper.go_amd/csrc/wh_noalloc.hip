// Device dequantisation that allocates nothing: wh_dequantize_noalloc.
//
// wh_dequantize stages the raw GGUF blocks, their re-laid-out planes and the
// float32 result in device buffers it allocates per call. This variant keeps
// all three in one file-scope device array (`scratch`), so a caller that cannot
// allocate (a serving loop, a harness that forbids hipMalloc) can still decode
// blocks on the device with the kernels' own bit-exact routine. The raw blocks
// are re-laid out by a kernel instead of a host staging image.
//
// Every call on a device shares that device's array and leaves the last call's
// contents in it: calls that overlap on one device race. Nothing in the array
// needs to start at zero (every byte a call reads it wrote first).
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <string>

#include "wh_device.h"
#include "wh_internal.h"

namespace wh {

namespace {

constexpr uint64_t SCRATCH_BYTES = 16ull << 20;  // 16 MiB per device
constexpr uint64_t MAX_ELEMS = 1ull << 20;       // fits every type: raw + planes + result <= 12 MiB

__device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
uint8_t *g_ptr[MAX_DEVICES];  // device address of `scratch` on each device, set once per device

// Device address of this device's copy of `scratch`; the first call on a
// device (made current here) asks the runtime for it.
int scratch_of(int32_t device, uint8_t **out) {
    if (device < 0 || device >= MAX_DEVICES) return fail(WH_ERR_INVALID, "dequantize_noalloc: bad device");
    std::lock_guard<std::mutex> lk(g_mu);
    WH_HIP(hipSetDevice(device));
    if (!g_ptr[device]) {
        void *p = nullptr;
        WH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(WH_ERR_HIP, "dequantize_noalloc: no device address for the scratch array");
        g_ptr[device] = (uint8_t *)p;
    }
    *out = g_ptr[device];
    return WH_OK;
}

uint64_t align256(uint64_t x) { return (x + 255) & ~255ull; }

// One row of nb raw GGUF blocks (internal/gguf/dequant.go:92-201 block layouts)
// scattered into the device planes the kernels read (wh_internal.h, DevMat):
// quants, scale words and Q5 high bits, bit for bit. F32/F16 rows become an
// f32 plane of nb * 32 values (F16 widened exactly, the tail zero).
__global__ void k_pack_row(uint32_t type, const uint8_t *raw, int32_t n, int32_t nb, uint8_t *qs, uint8_t *sc,
                           uint8_t *qh) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    if (type == WH_TYPE_F32 || type == WH_TYPE_F16) {
        float *o = (float *)qs + (size_t)b * 32;
        for (int j = 0; j < 32; j++) {
            const int c = b * 32 + j;
            float v = 0.0f;
            if (c < n) {
                if (type == WH_TYPE_F32) {
                    uint32_t u = 0;
                    for (int k = 0; k < 4; k++) u |= (uint32_t)raw[(size_t)c * 4 + k] << (8 * k);
                    v = __uint_as_float(u);
                } else {
                    v = h2f((uint16_t)(raw[(size_t)c * 2] | (raw[(size_t)c * 2 + 1] << 8)));
                }
            }
            o[j] = v;
        }
        return;
    }
    // bytes per block, offset of the high-bit word and of the quants within it, quant bytes
    int bb = 34, scw = 2, qho = -1, qso = 2, nq = 32;
    switch (type) {
    case WH_TYPE_Q4_0: bb = 18; scw = 2; qso = 2; nq = 16; break;
    case WH_TYPE_Q4_1: bb = 20; scw = 4; qso = 4; nq = 16; break;
    case WH_TYPE_Q5_0: bb = 22; scw = 2; qho = 2; qso = 6; nq = 16; break;
    case WH_TYPE_Q5_1: bb = 24; scw = 4; qho = 4; qso = 8; nq = 16; break;
    default: break;  // Q8_0
    }
    const uint8_t *s = raw + (size_t)b * bb;
    for (int k = 0; k < scw; k++) sc[(size_t)b * scw + k] = s[k];
    if (qho >= 0)
        for (int k = 0; k < 4; k++) qh[(size_t)b * 4 + k] = s[qho + k];
    for (int k = 0; k < nq; k++) qs[(size_t)b * nq + k] = s[qso + k];
}

}  // namespace

int dequantize_noalloc(uint32_t type, const void *raw, uint64_t nbytes, uint64_t n, float *out, int32_t device) {
    if (!out || (!raw && n)) return fail(WH_ERR_INVALID, "dequantize_noalloc: null buffer");
    if (n == 0) return WH_OK;
    if (n > MAX_ELEMS)
        return fail(WH_ERR_INVALID, "dequantize_noalloc: " + std::to_string(n) + " elements exceed the maximum of " +
                                        std::to_string(MAX_ELEMS) + " (16 MiB device scratch)");
    DevMat m;
    int rc = devmat_plan(m, type, 1, (int32_t)n);
    if (rc) return rc;
    const uint64_t need = gguf_row_bytes(type, n);
    if (nbytes < need)
        return fail(WH_ERR_INVALID, "dequantize_noalloc: short data got=" + std::to_string(nbytes) +
                                        " need=" + std::to_string(need));
    // scratch layout: raw blocks | quant plane | high bits | scale words | float result
    const uint64_t qs_bytes = (type == WH_TYPE_F32 || type == WH_TYPE_F16) ? (uint64_t)m.nb * 128
                              : type == WH_TYPE_Q8_0                       ? (uint64_t)m.nb * 32
                                                                           : (uint64_t)m.nb * 16;
    const uint64_t raw_off = 0, qs_off = align256(need), qh_off = align256(qs_off + qs_bytes);
    const uint64_t sc_off = align256(qh_off + (uint64_t)m.nb * 4), out_off = align256(sc_off + (uint64_t)m.nb * 4);
    if (out_off + n * sizeof(float) > SCRATCH_BYTES)
        return fail(WH_ERR_INVALID, "dequantize_noalloc: scratch too small");
    uint8_t *base = nullptr;
    if ((rc = scratch_of(device, &base))) return rc;
    WH_HIP(hipMemcpy(base + raw_off, raw, need, hipMemcpyHostToDevice));
    const int grid = (m.nb + 255) / 256;
    hipLaunchKernelGGL(k_pack_row, dim3(grid), dim3(256), 0, nullptr, type, base + raw_off, (int32_t)n, m.nb,
                       base + qs_off, base + sc_off, base + qh_off);
    WH_HIP(hipGetLastError());
    m.qs = base + qs_off;
    m.sc = (type == WH_TYPE_F32 || type == WH_TYPE_F16) ? nullptr : (void *)(base + sc_off);
    m.qh = (type == WH_TYPE_Q5_0 || type == WH_TYPE_Q5_1) ? (uint32_t *)(base + qh_off) : nullptr;
    m.alloc = nullptr;  // a view into the scratch array: nothing to free
    if ((rc = launch_dequant_rows(m, 0, 1, (float *)(base + out_off), nullptr))) return rc;
    WH_HIP(hipMemcpy(out, base + out_off, n * sizeof(float), hipMemcpyDeviceToHost));
    return WH_OK;
}

}  // namespace wh
