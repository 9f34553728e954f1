// Instantiation of the time-chunked fused SSM walk for bf16 storage (ssm_chunk.hpp).
#include "ssm_chunk.hpp"

namespace mqc {
template int ssm_chunk_launch<bf16_t>(const SsmArgs&, float*, hipStream_t);
}  // namespace mqc
