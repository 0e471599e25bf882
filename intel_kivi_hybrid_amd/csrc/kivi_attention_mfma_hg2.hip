// Matrix-core decode attention instantiated for Hq/Hkv = 2.
#include "kivi_attention_mfma.hpp"

namespace kivi {

int launch_attention_mfma_hg2(const AttnLaunch& a, hipStream_t st) { return launch_d<2>(a, st); }

}  // namespace kivi
