// Batched persistent forward for Q4_1 weights (kernel in wh_batch_kernel.h).
#include "wh_batch_kernel.h"

namespace wh {
namespace batch {
int launch_q4_1(int grid, const BArgs &a, hipStream_t st) { return launch_type<3>(grid, a, st); }
int warm_q4_1(int d) { return warm_type<3>(d); }
}  // namespace batch
}  // namespace wh
