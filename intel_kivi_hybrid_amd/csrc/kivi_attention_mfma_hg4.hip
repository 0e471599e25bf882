// Matrix-core decode attention instantiated for Hq/Hkv = 4.
#include "kivi_attention_mfma.hpp"

namespace kivi {

int launch_attention_mfma_hg4(const AttnLaunch& a, hipStream_t st) { return launch_d<4>(a, st); }

}  // namespace kivi
