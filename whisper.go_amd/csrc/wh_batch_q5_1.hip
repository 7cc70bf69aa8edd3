// Batched persistent forward for Q5_1 weights (kernel in wh_batch_kernel.h).
#include "wh_batch_kernel.h"

namespace wh {
namespace batch {
int launch_q5_1(int grid, const BArgs &a, hipStream_t st) { return launch_type<7>(grid, a, st); }
int warm_q5_1(int d) { return warm_type<7>(d); }
}  // namespace batch
}  // namespace wh
