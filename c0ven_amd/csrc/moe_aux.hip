// Decoding a matrix in the device layout back to fp32 with the kernels' own loaders (units.h): the check that the
// layout and the field extraction give the format's values (moe_dequantize).
#include <hip/hip_runtime.h>

#include "aux.h"
#include "iq3s_grid.h"
#include "units.h"

namespace c0ven {

__device__ __constant__ static const uint32_t kGridAux[512] = {C0VEN_IQ3S_GRID_VALUES};

// Grid: one work-group of 64 (a wave) per tile; lane l writes row rt * 64 + l, all its units. The values are
// formed as ggml's dequantize_row_* forms them: Q8_0 d q; Q4_K (d sc) q - (dmin m); IQ3_S (d (1 + 2 s)) (sign grid);
// IQ3_XXS and IQ2_S with the grid the caller's codebooks hold.
__global__ void __launch_bounds__(64) moe_dequant(const uint8_t *mat, uint32_t type, uint32_t rows, uint32_t k,
                                                  const uint8_t *codebooks, float *out) {
  __shared__ uint32_t grid[2048];
  if (type == QT_IQ3_S) {
    for (uint32_t i = threadIdx.x; i < 512; i += 64) grid[i] = kGridAux[i];
  } else if (type == QT_IQ3_XXS || type == QT_IQ2_S) {
    const uint32_t *src = (const uint32_t *)(codebooks + (type == QT_IQ2_S ? QGRID_IQ2S : QGRID_IQ3XXS));
    for (uint32_t i = threadIdx.x; i < (type == QT_IQ2_S ? 2048u : 256u); i += 64) grid[i] = src[i];
  }
  __syncthreads();
  const uint32_t U = units_of(k), rt = blockIdx.x, lane = threadIdx.x, nl = kTileRows * U;
  const uint32_t row = rt * kTileRows + lane;
  const uint8_t *tile = mat + (uint64_t)rt * tile_bytes(type, U);
  const bool live = row < rows;
  for (uint32_t u = 0; u < U; u++) {
  const uint32_t idx = pair_idx(lane, u), nv = min(kUnit, k - u * kUnit);  // nv: the unit's values (partial last)
  float *o = out + (uint64_t)row * k + u * kUnit;
  if (q8_family(type)) {  // a code and its 32-value block's scale: d q, d kvalues[nibble], d (q - 1)
    UnitQ8_0 w;
    if (type == QT_IQ4_NL)
      static_cast<UnitIQ4_NL &>(w).load(tile, idx, nl);
    else if (type == QT_Q2_0)
      static_cast<UnitQ2_0 &>(w).load(tile, idx, nl);
    else
      w.load(tile, idx, nl);
    if (live)
      for (uint32_t i = 0; i < nv; i++) o[i] = __fmul_rn(w.d[i / 32], (float)(int8_t)(w.q[i / 4] >> (8 * (i % 4))));
  } else if (type == QT_Q4_K) {
    UnitQ4_K w;
    w.load(tile, idx, nl);
    if (live)
      for (int wd = 0; wd < 32; wd++)
        for (int i = 0; i < 4; i++) {
          const int c = wd / 8, v = 64 * c + 4 * (wd % 8) + i;
          const float dl = __fmul_rn(w.d, (float)w.sc[2 * c]), ml = __fmul_rn(w.dmin, (float)w.mn[2 * c]);
          const float dh = __fmul_rn(w.d, (float)w.sc[2 * c + 1]), mh = __fmul_rn(w.dmin, (float)w.mn[2 * c + 1]);
          o[v] = __fsub_rn(__fmul_rn(dl, (float)((w.lo[wd] >> (8 * i)) & 0xff)), ml);
          o[v + 32] = __fsub_rn(__fmul_rn(dh, (float)((w.hi[wd] >> (8 * i)) & 0xff)), mh);
        }
  } else if (type == QT_Q5_K) {  // (d sc) q - (dmin m), q 0..31
    UnitQ5_K w;
    w.load(tile, idx, nl);
    if (live)
      for (int wd = 0; wd < 32; wd++)
        for (int i = 0; i < 4; i++) {
          const int c = wd / 8, v = 64 * c + 4 * (wd % 8) + i;
          const float dl = __fmul_rn(w.d, (float)w.sc[2 * c]), ml = __fmul_rn(w.dmin, (float)w.mn[2 * c]);
          const float dh = __fmul_rn(w.d, (float)w.sc[2 * c + 1]), mh = __fmul_rn(w.dmin, (float)w.mn[2 * c + 1]);
          o[v] = __fsub_rn(__fmul_rn(dl, (float)((w.lo[wd] >> (8 * i)) & 0xff)), ml);
          o[v + 32] = __fsub_rn(__fmul_rn(dh, (float)((w.hi[wd] >> (8 * i)) & 0xff)), mh);
        }
  } else if (type == QT_Q6_K) {  // (d sc) (q - 32)
    UnitQ6_K w;
    w.load(tile, idx, nl);
    if (live)
      for (int i = 0; i < 256; i++)
        o[i] = __fmul_rn(__fmul_rn(w.d, (float)w.sc[i / 16]), (float)(int8_t)(w.w[i / 4] >> (8 * (i % 4))));
  } else if (type == QT_IQ4_XS) {  // (d (ls - 32)) kvalues[nibble]
    UnitIQ4_XS w;
    w.load(tile, idx, nl);
    if (live)
      for (int i = 0; i < 256; i++)
        o[i] = __fmul_rn(__fmul_rn(w.d, (float)w.ls[i / 32]), (float)(int8_t)(w.q[i / 4] >> (8 * (i % 4))));
  } else if (type == QT_IQ3_XXS) {  // (d (0.5 + s)) 0.5, times the signed grid value
    UnitIQ3_XXS w;
    w.load(tile, idx, nl, grid);
    if (live)
      for (int i = 0; i < 256; i++) {
        const float db = __fmul_rn(__fmul_rn(w.d, 0.5f + (float)((w.ls[i / 32] - 1) / 2)), 0.5f);
        o[i] = __fmul_rn(db, (float)(int8_t)(w.w[i / 4] >> (8 * (i % 4))));
      }
  } else if (type == QT_IQ2_S) {  // (d (0.5 + s)) 0.25 for each half sub-block, times the signed grid value
    UnitIQ2_S w;
    w.load(tile, idx, nl, grid);
    if (live)
      for (int i = 0; i < 256; i++) {
        const float db = __fmul_rn(__fmul_rn(w.d, 0.5f + (float)((w.ls[i / 16] - 1) / 2)), 0.25f);
        o[i] = __fmul_rn(db, (float)(int8_t)(w.w[i / 4] >> (8 * (i % 4))));
      }
  } else {
    UnitIQ3_S w;
    w.load(tile, idx, nl, grid);
    if (live)
      for (int i = 0; i < 256; i++) {
        const float db = __fmul_rn(w.d, (float)w.ls[i / 32]);
        o[i] = __fmul_rn(db, (float)(int8_t)(w.w[i / 4] >> (8 * (i % 4))));
      }
  }
  }
}

}  // namespace c0ven
