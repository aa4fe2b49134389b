// RMSNorm forward launcher instantiated for __bf16 storage (kernels in rmsnorm_impl.hpp).
#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {
template bool launch_fwd<__bf16>(const FwdArgs&);
}  // namespace rmsnorm
}  // namespace pt
