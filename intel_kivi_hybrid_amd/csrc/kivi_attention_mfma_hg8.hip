// Matrix-core decode attention instantiated for Hq/Hkv = 8, fp32 residual ring.
#include "kivi_attention_mfma.hpp"

namespace kivi {

int launch_attention_mfma_hg8(const AttnLaunch& a, hipStream_t st) {
    return launch_d<8, false>(a, st);
}

}  // namespace kivi
