// Packed decode attention on the gfx950 matrix cores (placeholder: not yet built).
#include "decode_common.hpp"

namespace lf {

int launch_decode_mfma(const DecodeParams& p, hipStream_t stream, bool* handled) {
    (void)p;
    (void)stream;
    *handled = false;
    return LF_OK;
}

}  // namespace lf
