// Shared definitions of the C facade's opaque handles.
#pragma once

#include "kim-kv/engine/engine_kv.h"
#include "kim-kv/runtime/kv_cache_manager.h"

#include <memory>

struct kimkv_engine {
    std::unique_ptr<kimkvcache::EngineKvBackend> backend;
};

// A manager handle either owns its KvCacheManager (kimkv_manager_create) or
// views the one inside a kimkv_cache (kimkv_cache_manager).
struct kimkv_manager {
    std::unique_ptr<kimkvcache::KvCacheManager> owned;
    kimkvcache::KvCacheManager* m{nullptr};
};
