// Instantiation of the fused quaternion SSM backward for bf16 storage (ssm_bwd.hpp).
#include "ssm_bwd.hpp"

namespace mqc {
template int launch_ssm_bwd<bf16_t>(const SsmBwdArgs&, hipStream_t);
}  // namespace mqc
