// RMSNorm backward launcher instantiated for _Float16 storage (kernels in rmsnorm_impl.hpp).
#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {
template bool launch_bwd<_Float16>(const BwdArgs&);
}  // namespace rmsnorm
}  // namespace pt
