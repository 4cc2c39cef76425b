// The decode kernel's type sets 8 - 15 (the codebook types) with the hyper-connection mix and combine: instantiated
// here so that they compile in parallel with the others.
#define C0VEN_DECODE_HC_IQ2_SETS
#include "moe_decode.hip"
