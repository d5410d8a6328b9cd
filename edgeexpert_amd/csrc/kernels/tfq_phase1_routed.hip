// tfq_phase1_routed.hip — routed decode phase 1 with the router's top-k selection folded in,
// at 4, 3 and 2 bits.
#include "entry_points.hpp"

TFQ_Q4_TABLE(TFQ_PHASE1_ROUTED)
TFQ_Q4_TABLE(TFQ_PHASE1_ROUTED_B)
