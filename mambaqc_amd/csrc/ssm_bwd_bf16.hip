// Instantiation of the fused quaternion SSM backward for bf16 storage (ssm_bwd.hpp, ssm_bwd_chunk.hpp).
#include "ssm_bwd_chunk.hpp"

namespace mqc {
template int launch_ssm_bwd<bf16_t>(const SsmBwdArgs&, hipStream_t);
template int ssm_bwd_chunked_launch<bf16_t>(const SsmBwdArgs&, float*, hipStream_t);
}  // namespace mqc
