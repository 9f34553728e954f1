// Instantiation of the time-chunked fused SSM walk for f32 storage (ssm_chunk.hpp).
#include "ssm_chunk.hpp"

namespace mqc {
template int ssm_chunk_launch<float>(const SsmArgs&, float*, hipStream_t);
}  // namespace mqc
