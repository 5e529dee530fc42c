// pending.hip -- launchers whose kernels are not written yet report an error.
#include "common.hpp"
#include "kernels.hpp"
namespace gfh {
#define PENDING(name) return set_error(GFH_COMPUTATION_FAILED, name ": kernel not built yet")
int launch_qlinear_i8(const QLinearDesc &, hipStream_t) { PENDING("qlinear"); }
int launch_gemv_f32(const float *, const float *, float *, int64_t, int64_t, int64_t, hipStream_t) { PENDING("gemv_f32"); }
int launch_gemv_w8(const float *, const int8_t *, const float *, const int8_t *, float *, int64_t, int64_t, int64_t, hipStream_t) { PENDING("gemv_w8"); }
int launch_softmax_lastdim(const float *, float *, int64_t, int64_t, hipStream_t) { PENDING("softmax"); }
int launch_sdpa(const SdpaDesc &, hipStream_t) { PENDING("sdpa"); }
}
