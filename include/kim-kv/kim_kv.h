// Umbrella header of the CPU-side API (the reference's include/kim-kv/kim_kv.h:1-22).
// HIP entry points stay opt-in through kim-kv/hip/ and kimkv_hip.h.  Not
// provided by this build, so not included: kim-kv/fixed/fixed_page_manager.h
// (the fixed-size page strategy is outside the heterogeneous data path).
#pragma once

#include "kim-kv/core/block_table.h"
#include "kim-kv/core/kv_layout.h"
#include "kim-kv/core/page_handle.h"
#include "kim-kv/core/page_pool.h"
#include "kim-kv/core/page_state.h"
#include "kim-kv/core/page_types.h"
#include "kim-kv/engine/engine_kv.h"
#include "kim-kv/engine/generation.h"
#include "kim-kv/engine/iteration_scheduler.h"
#include "kim-kv/model/tinyllama_config.h"
#include "kim-kv/reference/kv_reference.h"
#include "kim-kv/runtime/kv_cache_manager.h"
#include "kim-kv/runtime/page_lease.h"
#include "kim-kv/runtime/promotion.h"
#include "kim-kv/runtime/token_reservation.h"
