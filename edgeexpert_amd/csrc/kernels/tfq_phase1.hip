// tfq_phase1.hip — routed decode phase 1 (gate/up/GeGLU of the selected experts) at
// 4, 3 and 2 bits, full and subset forms.
#include "entry_points.hpp"

TFQ_Q4_TABLE(TFQ_PHASE1)
TFQ_Q4_TABLE(TFQ_PHASE1_B)
