// Matrix-core decode attention instantiated for Hq/Hkv = 1, fp32 residual ring;
// also the LDS size query of every matrix-core shape.
#include "kivi_attention_mfma.hpp"

namespace kivi {

int launch_attention_mfma_hg1(const AttnLaunch& a, hipStream_t st) {
    return launch_d<1, false>(a, st);
}

namespace {
template <int HG>
int lds_for(int D, int G, int NG) {
    if (G != 32 && G != 64) return -1;
    switch (D) {
        case 64: return G == 32 ? Shape<HG, 64, 32>::lds(NG) : Shape<HG, 64, 64>::lds(NG);
        case 128: return G == 32 ? Shape<HG, 128, 32>::lds(NG) : Shape<HG, 128, 64>::lds(NG);
        case 256: return G == 32 ? Shape<HG, 256, 32>::lds(NG) : Shape<HG, 256, 64>::lds(NG);
        default: return -1;
    }
}
}  // namespace

int attention_mfma_lds_bytes(int HG, int D, int G, int NG) {
    switch (HG) {
        case 1: return lds_for<1>(D, G, NG);
        case 2: return lds_for<2>(D, G, NG);
        case 4: return lds_for<4>(D, G, NG);
        case 8: return lds_for<8>(D, G, NG);
        default: return -1;
    }
}

}  // namespace kivi
