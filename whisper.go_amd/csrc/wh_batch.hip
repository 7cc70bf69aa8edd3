// Dispatch of the batched persistent forward to the instantiation for the
// model's weight type (wh_batch_q*.hip, kernel in wh_batch_kernel.h).
#include <hip/hip_runtime.h>

#include "wh_batch.h"
#include "wh_internal.h"

namespace wh {
namespace batch {

int launch_q4_0(int grid, const BArgs &a, hipStream_t st);
int launch_q4_1(int grid, const BArgs &a, hipStream_t st);
int launch_q5_0(int grid, const BArgs &a, hipStream_t st);
int launch_q5_1(int grid, const BArgs &a, hipStream_t st);
int launch_q8_0(int grid, const BArgs &a, hipStream_t st);
int warm_q4_0(int d);
int warm_q4_1(int d);
int warm_q5_0(int d);
int warm_q5_1(int d);
int warm_q8_0(int d);

// Code objects of the batched forward for a model of weight type `type` and width d.
int warm(uint32_t type, int d) {
    switch (type) {
    case 2: return warm_q4_0(d);
    case 3: return warm_q4_1(d);
    case 6: return warm_q5_0(d);
    case 7: return warm_q5_1(d);
    case 8: return warm_q8_0(d);
    default: return WH_OK;
    }
}

int launch(uint32_t type, int grid, const BArgs &a, hipStream_t st) {
    switch (type) {
    case 2: return launch_q4_0(grid, a, st);
    case 3: return launch_q4_1(grid, a, st);
    case 6: return launch_q5_0(grid, a, st);
    case 7: return launch_q5_1(grid, a, st);
    case 8: return launch_q8_0(grid, a, st);
    default: return fail(WH_ERR_UNSUPPORTED, "batched persistent forward: unsupported weight type");
    }
}

}  // namespace batch
}  // namespace wh
