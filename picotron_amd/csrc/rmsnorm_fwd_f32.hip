// RMSNorm forward launcher instantiated for float storage (kernels in rmsnorm_impl.hpp).
#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {
template bool launch_fwd<float>(const FwdArgs&);
}  // namespace rmsnorm
}  // namespace pt
