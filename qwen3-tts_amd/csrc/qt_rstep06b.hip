// qt_rstep06b.hip — the role-specialised decode step of qt_rstep.hip built for the 0.6B
// geometry with bf16 weights (bf16 MFMA against three exact bf16 activation planes;
// namespace ps::rs06b, entry points qt_rstep06b_* / qt_launch_rstep06b*).
#define QT_RS_SMALL 1
#define QT_RS_BF16 1
#include "qt_rstep.hip"
