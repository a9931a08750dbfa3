#include "common.hpp"
namespace luxhip {
bool qgemm_small_supported(const QArgs&) { return false; }
hipError_t launch_qgemm_small(const QArgs&, hipStream_t) { return hipErrorInvalidValue; }
bool w4a8_supported(const QArgs&) { return false; }
hipError_t launch_w4a8(const QArgs&, hipStream_t) { return hipErrorInvalidValue; }
}
