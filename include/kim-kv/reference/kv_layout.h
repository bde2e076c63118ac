// Compatibility header of the reference (include/kim-kv/reference/kv_layout.h):
// the layout lives in core/kv_layout.h.
#pragma once

#include "kim-kv/core/kv_layout.h"
