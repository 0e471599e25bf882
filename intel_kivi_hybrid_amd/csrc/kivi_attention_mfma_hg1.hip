// Matrix-core decode attention instantiated for Hq/Hkv = 1.
#include "kivi_attention_mfma.hpp"

namespace kivi {

int launch_attention_mfma_hg1(const AttnLaunch& a, hipStream_t st) { return launch_d<1>(a, st); }

}  // namespace kivi
