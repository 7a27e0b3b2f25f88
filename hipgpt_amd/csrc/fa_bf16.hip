// fa_bf16.hip -- bf16-input / fp32-accumulate MFMA attention (not built yet).
#include "common.h"
#include "kernels.h"

namespace hipgpt {

bool fa_bf16_supported(int) { return false; }

hipError_t launch_fa_bf16(const AttnArgs&, bool, hipStream_t) { return hipErrorNotSupported; }

}  // namespace hipgpt
