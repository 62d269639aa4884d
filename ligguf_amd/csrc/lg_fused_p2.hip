/* lg_fused_p2.hip -- part 2 of the fused step's variant table (the
 * variants of each part compile in a translation unit of their own) */
#define LG_FUSED_PART 2
#include "lg_fused.hip"
