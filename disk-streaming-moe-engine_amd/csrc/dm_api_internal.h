// dm_api_internal.h -- helpers shared by the C ABI's translation units.
#ifndef DM_API_INTERNAL_H
#define DM_API_INTERNAL_H

#include <stddef.h>

#include "../../include/dismoen_hip.h"

namespace dm {

// CONFIG_ERROR unless the 4-bit layer dimensions are supported (group size
// in {32, 64, 128, 256}, H / I / I_sh multiples of 128, E <= 2048, K <= 32).
// Callers run it before any size arithmetic or allocation on the dims.
int api_moe_dims_check(const dmh_moe_dims* d, int layer, char* err, size_t errlen);

}  // namespace dm

#endif
