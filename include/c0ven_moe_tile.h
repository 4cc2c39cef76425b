/* The records the routing kernels write and the expert kernels read.
 *
 * Replaces the reference's shared/moe_tile.h: MoeTile (:11-18, 16 B), MoeGroup (:23-33, 40 B), MOE_TILE (:9),
 * MOE_GROUP_MAX (:21), MOE_WG_ROWS (:38). Same fields, same sizes, same meaning:
 *   MoeTile  - up to MOE_TILE consecutive rows of the expert-ordered activations, all routed to one expert
 *              (the prefill path's grouped GEMM takes one tile per work-group row block);
 *   MoeGroup - one expert and the assignments (token * n_used + rank) of a decode step that route to it, so its
 *              weights are read once for all of them; an expert with more than MOE_GROUP_MAX assignments takes a
 *              group for each MOE_GROUP_MAX of them. */
#ifndef C0VEN_MOE_TILE_H
#define C0VEN_MOE_TILE_H

#include <stdint.h>

#include "c0ven_quant.h"

#define MOE_TILE 64 /* a multiple of 32 */

typedef struct {
  uint32_t expert;
  uint32_t slot;  /* where the expert's weights sit: its index in the layer's resident experts */
  uint32_t start; /* first row of the expert-ordered activations */
  uint32_t count; /* rows, 1 .. MOE_TILE */
} MoeTile;

#define MOE_GROUP_MAX 8

typedef struct {
  int32_t slot;                 /* the expert's slot; the shared expert is slot n_expert */
  uint32_t n;                   /* assignments, 1 .. MOE_GROUP_MAX */
  uint32_t asg[MOE_GROUP_MAX];  /* token * n_used + rank; the shared expert's are n_tok * n_used + token */
} MoeGroup;

/* Rows one decode work-group computes of a group's expert. */
#define MOE_WG_ROWS 32

#ifdef __cplusplus
static_assert(sizeof(MoeTile) == 16, "MoeTile layout");
static_assert(sizeof(MoeGroup) == 40, "MoeGroup layout");
#else
_Static_assert(sizeof(MoeTile) == 16, "MoeTile layout");
_Static_assert(sizeof(MoeGroup) == 40, "MoeGroup layout");
#endif

#endif
