// Instantiation of the fused quaternion SSM for f16 storage (ssm_scan.hpp).
#include "ssm_scan.hpp"

namespace mqc {
template int launch_ssm<f16_t, MODE_DL>(const SsmArgs&, hipStream_t);
template int launch_ssm<f16_t, MODE_Q>(const SsmArgs&, hipStream_t);
}  // namespace mqc
