// Backward multi-pathway attention (placeholder until the kernels land).
#include "mpattn_common.h"

namespace mpattn {
int64_t bwd_workspace_bytes(int B, int H, int L, int D) {
    (void)D;
    return (int64_t)B * H * L * 4;
}
hipError_t launch_bwd(const mpattn_bwd_params& p, hipStream_t stream) {
    (void)p; (void)stream;
    return hipErrorInvalidValue;
}
hipError_t launch_fwd32(const mpattn_fwd_params& p, hipStream_t stream) {
    (void)p; (void)stream;
    return hipErrorInvalidValue;
}
}  // namespace mpattn
