#include "dispatch.hpp"
namespace clove {
clove_status_t launch_gemm_int8(const Int8Args&, hipStream_t) { return CLOVE_ERR_LAUNCH; }
clove_status_t launch_gemm_int4(const Int4Args&, hipStream_t) { return CLOVE_ERR_LAUNCH; }
clove_status_t launch_w4a16(const W4A16Args&, hipStream_t) { return CLOVE_ERR_LAUNCH; }
}
