// Instantiation of the fused quaternion SSM for f32 storage (ssm_scan.hpp).
#include "ssm_scan.hpp"

namespace mqc {
template int launch_ssm<float, MODE_DL>(const SsmArgs&, hipStream_t);
template int launch_ssm<float, MODE_Q>(const SsmArgs&, hipStream_t);
}  // namespace mqc
