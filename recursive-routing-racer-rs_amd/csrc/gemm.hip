// gemm.hip -- prefill dequant-GEMM (MFMA).  Placeholder until the MFMA kernel lands.
#include "device_common.h"
#include "internal.h"

namespace rrr {

hipError_t launch_gemm_bf16(const uint16_t *, const uint8_t *, uint64_t, uint32_t, float *, uint32_t, uint32_t,
                            uint32_t, hipStream_t)
{
    return hipErrorNotSupported;
}

}  // namespace rrr
