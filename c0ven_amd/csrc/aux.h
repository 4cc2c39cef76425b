#pragma once

#include <stdint.h>

namespace c0ven {

__global__ void moe_dequant(const uint8_t *mat, uint32_t type, uint32_t rows, uint32_t k, float *out);

}  // namespace c0ven
