// The decode kernel's type sets 1 - 7 with the hyper-connection mix and combine (moe_forward_hc): instantiated here so
// that they compile in parallel with the others.
#define C0VEN_DECODE_HC_SETS
#include "moe_decode.hip"
