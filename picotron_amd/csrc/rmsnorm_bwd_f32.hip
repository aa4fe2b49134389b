// RMSNorm backward launcher instantiated for float storage (kernels in rmsnorm_impl.hpp).
#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {
template bool launch_bwd<float>(const BwdArgs&);
}  // namespace rmsnorm
}  // namespace pt
