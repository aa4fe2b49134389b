// RMSNorm forward launcher instantiated for _Float16 storage (kernels in rmsnorm_impl.hpp).
#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {
template bool launch_fwd<_Float16>(const FwdArgs&);
}  // namespace rmsnorm
}  // namespace pt
