// Status reporting shared by the library's C entry points: records the
// static detail text that hkbs_last_error() returns on the calling thread.
#pragma once

#include "../../include/hkbs_pmpnn.h"

namespace hkbs {

hkbs_status report_error(hkbs_status code, const char* detail);

}  // namespace hkbs
