// fa_prefill.hip -- causal prefill / large verify blocks on gfx950 MFMA.
#include "fa_device.hpp"

namespace sixi {

hipError_t launch_prefill(const FaArgs&, int, int, int, hipStream_t) { return hipErrorNotSupported; }

}  // namespace sixi
