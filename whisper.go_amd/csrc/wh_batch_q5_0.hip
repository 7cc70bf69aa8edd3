// Batched persistent forward for Q5_0 weights (kernel in wh_batch_kernel.h).
#include "wh_batch_kernel.h"

namespace wh {
namespace batch {
int launch_q5_0(int grid, const BArgs &a, hipStream_t st) { return launch_type<6>(grid, a, st); }
int warm_q5_0(int d) { return warm_type<6>(d); }
}  // namespace batch
}  // namespace wh
