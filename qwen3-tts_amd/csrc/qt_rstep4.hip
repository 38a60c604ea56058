// qt_rstep4.hip — the role-specialised decode step of qt_rstep.hip built for the 1.7B
// geometry with q4_0 weights (integer MFMA on the exact int8 activation planes, the f16
// block scales applied to each block's exact sums; namespace ps::rs4, entry points
// qt_rstep4_* / qt_launch_rstep4).
#define QT_RS_Q4 1
#include "qt_rstep.hip"
