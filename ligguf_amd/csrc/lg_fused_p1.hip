/* lg_fused_p1.hip -- part 1 of the fused step's variant table (the
 * variants of each part compile in a translation unit of their own) */
#define LG_FUSED_PART 1
#include "lg_fused.hip"
