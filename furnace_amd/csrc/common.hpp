// Shared host-side helpers of the engine library.
#pragma once
#include "../../include/furnace_hip.h"

// Record a printf-style message as frn_last_error() for this thread and
// return st.
frn_status frn_fail(frn_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
