#pragma once

#include <stdint.h>

namespace c0ven {

__global__ void moe_dequant(const uint8_t *mat, uint32_t type, uint32_t rows, uint32_t k, const uint8_t *codebooks,
                            float *out);

}  // namespace c0ven
