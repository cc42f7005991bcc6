/* The C ABI of libtinybrain_hip as one Swift module (CTinyBrainHIP). */
#include "../../../include/tinybrain_hip.h"
