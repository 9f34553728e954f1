// Instantiation of the fused quaternion SSM backward for f16 storage (ssm_bwd.hpp, ssm_bwd_chunk.hpp).
#include "ssm_bwd_chunk.hpp"

namespace mqc {
template int launch_ssm_bwd<f16_t>(const SsmBwdArgs&, hipStream_t);
template int ssm_bwd_chunked_launch<f16_t>(const SsmBwdArgs&, float*, hipStream_t);
}  // namespace mqc
