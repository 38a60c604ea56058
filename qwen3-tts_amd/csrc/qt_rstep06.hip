// qt_rstep06.hip — the role-specialised decode step of qt_rstep.hip built for the 0.6B
// geometry (hidden 1024, intermediate 3072; namespace ps::rs06, entry points
// qt_rstep06_* / qt_launch_rstep06).
#define QT_RS_SMALL 1
#include "qt_rstep.hip"
