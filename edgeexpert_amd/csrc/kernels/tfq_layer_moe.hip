// tfq_layer_moe.hip — the decoder layer's feed-forward launches with the shared expert
// (int4 or int8) folded in (4-bit routed experts): phase 1 + shared gate/up/act,
// phase 2 + shared down.
#include "entry_points.hpp"

TFQ_Q4_TABLE(TFQ_PHASE1_SHARED)
TFQ_PHASE2_SHARED(1)
TFQ_PHASE2_SHARED(2)
TFQ_PHASE2_SHARED(3)
TFQ_PHASE2_SHARED(4)

// the (routed, int8 shared) row shapes that d = 64..4096 select (seg_shape_fit(d/32, 2),
// seg_shape(d/16, 4))
TFQ_PHASE1_SHARED8(2, 1, 4, 1)
TFQ_PHASE1_SHARED8(4, 1, 8, 1)
TFQ_PHASE1_SHARED8(8, 1, 16, 1)
TFQ_PHASE1_SHARED8(8, 3, 64, 1)
TFQ_PHASE1_SHARED8(16, 1, 32, 1)
TFQ_PHASE1_SHARED8(16, 3, 64, 2)
TFQ_PHASE1_SHARED8(32, 1, 64, 1)
TFQ_PHASE1_SHARED8(32, 3, 64, 3)
TFQ_PHASE1_SHARED8(64, 1, 64, 2)
TFQ_PHASE1_SHARED8(64, 2, 64, 4)
TFQ_Q8_TABLE(TFQ_PHASE2_SHARED8_P1)
TFQ_Q8_TABLE(TFQ_PHASE2_SHARED8_P2)
TFQ_Q8_TABLE(TFQ_PHASE2_SHARED8_P3)
TFQ_Q8_TABLE(TFQ_PHASE2_SHARED8_P4)
