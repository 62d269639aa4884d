/* lg_fused_p3.hip -- part 3 of the fused step's variant table (the
 * variants of each part compile in a translation unit of their own) */
#define LG_FUSED_PART 3
#include "lg_fused.hip"
