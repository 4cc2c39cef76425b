// The decode kernel's type sets that hold the codebook types (IQ3_XXS, IQ2_S): instantiated here so that the two
// halves of the set list compile in parallel.
#define C0VEN_DECODE_IQ2_SETS
#include "moe_decode.hip"
