// RMSNorm backward launcher instantiated for __bf16 storage (kernels in rmsnorm_impl.hpp).
#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {
template bool launch_bwd<__bf16>(const BwdArgs&);
}  // namespace rmsnorm
}  // namespace pt
