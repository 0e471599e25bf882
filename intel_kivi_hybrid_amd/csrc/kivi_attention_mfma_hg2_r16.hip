// Matrix-core decode attention instantiated for Hq/Hkv = 2, bf16/fp16
// residual ring.
#include "kivi_attention_mfma.hpp"

namespace kivi {

int launch_attention_mfma_hg2_r16(const AttnLaunch& a, hipStream_t st) {
    return launch_d<2, true>(a, st);
}

}  // namespace kivi
