// tfq_layer_moe.hip — the decoder layer's feed-forward launches with the int4 shared
// expert folded in (4-bit routed experts): phase 1 + shared gate/up/act, phase 2 +
// shared down.
#include "entry_points.hpp"

TFQ_Q4_TABLE(TFQ_PHASE1_SHARED)
TFQ_PHASE2_SHARED(1)
TFQ_PHASE2_SHARED(2)
TFQ_PHASE2_SHARED(3)
TFQ_PHASE2_SHARED(4)
