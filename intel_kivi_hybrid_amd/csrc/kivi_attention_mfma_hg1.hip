// Matrix-core decode attention instantiated for Hq/Hkv = 1, fp32 residual ring.
#include "kivi_attention_mfma.hpp"

namespace kivi {

int launch_attention_mfma_hg1(const AttnLaunch& a, hipStream_t st) {
    return launch_d<1, false>(a, st);
}

}  // namespace kivi
