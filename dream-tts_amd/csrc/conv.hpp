// Channels-last conv entry points shared by the C ABI and the codec driver.
#pragma once

#include <cstring>

#include "common.hpp"

namespace dtts {

// "mfma" when the tiled matrix-core kernel takes the descriptor's shape, else "direct".
const char *conv_path_name(const dtts_conv_desc *d);
int conv1d_nlc_f16(const dtts_conv_desc *d, hipStream_t stream);

}  // namespace dtts
