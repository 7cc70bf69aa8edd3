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
