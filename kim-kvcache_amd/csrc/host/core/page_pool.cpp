// PagePool: slot + generation handles over a LIFO free list
// (semantics of src/core/page_pool.cpp:8-179 in the reference: slots are
// handed out 0, 1, 2, ... from a fresh pool, a released slot is the next one
// reused, generation 0 is never issued).
#include "kim-kv/core/page_pool.h"

#include <stdexcept>

namespace kimkvcache {
namespace {

std::uint32_t bumpGeneration(std::uint32_t g) noexcept
{
    ++g;
    return g == PageHandle::kInvalidGeneration ? 1u : g;
}

}  // namespace

PagePool::PagePool(PageKind kind, std::uint32_t capacity) : kind_(kind), capacity_(capacity)
{
    if (!isKnownPageKind(kind)) throw std::invalid_argument("PagePool kind must be Micro or Extent");
    if (capacity == 0) throw std::invalid_argument("PagePool capacity must be greater than zero");
    slots_.resize(capacity);
    free_.reserve(capacity);
    for (std::uint32_t s = capacity; s > 0; --s) free_.push_back(s - 1);
}

PageAllocationResult PagePool::allocate()
{
    std::lock_guard<std::mutex> lock(mutex_);
    if (free_.empty()) {
        ++failed_allocations_;
        return {PagePoolError::Exhausted, PageHandle::invalid()};
    }
    std::uint32_t const slot = free_.back();
    if (slot >= slots_.size() || slots_[slot].allocated || allocated_ >= capacity_) {
        throw std::logic_error("PagePool invariant violation in allocate");
    }
    free_.pop_back();
    Slot& s = slots_[slot];
    s.generation = bumpGeneration(s.generation);
    s.allocated = true;
    ++allocated_;
    ++allocations_;
    return {PagePoolError::None, PageHandle{kind_, slot, s.generation}};
}

PagePoolError PagePool::release(PageHandle handle)
{
    std::lock_guard<std::mutex> lock(mutex_);
    PagePoolError const v = validateLocked(handle);
    if (v != PagePoolError::None) {
        ++rejected_releases_;
        return v;
    }
    if (allocated_ == 0 || free_.size() >= slots_.size()) {
        throw std::logic_error("PagePool invariant violation in release");
    }
    free_.push_back(handle.slot);
    slots_[handle.slot].allocated = false;
    --allocated_;
    ++releases_;
    return PagePoolError::None;
}

PagePoolError PagePool::validate(PageHandle handle) const
{
    std::lock_guard<std::mutex> lock(mutex_);
    return validateLocked(handle);
}

PagePoolError PagePool::validateLocked(PageHandle handle) const noexcept
{
    if (!handle.isStructurallyValid()) return PagePoolError::InvalidHandle;
    if (handle.kind != kind_) return PagePoolError::WrongKind;
    if (handle.slot >= slots_.size()) return PagePoolError::OutOfRange;
    Slot const& s = slots_[handle.slot];
    // A reused slot reports the stale handle as stale, not as already free.
    if (handle.generation != s.generation) return PagePoolError::StaleGeneration;
    if (!s.allocated) return PagePoolError::AlreadyFree;
    return PagePoolError::None;
}

PagePoolSnapshot PagePool::snapshot() const
{
    std::lock_guard<std::mutex> lock(mutex_);
    return PagePoolSnapshot{kind_, capacity_, static_cast<std::uint32_t>(free_.size()), allocated_,
                            allocations_, releases_, failed_allocations_, rejected_releases_};
}

bool PagePool::checkInvariants() const
{
    std::lock_guard<std::mutex> lock(mutex_);
    if (slots_.size() != capacity_ || free_.size() + allocated_ != capacity_) return false;
    std::vector<std::uint8_t> on_free_list(slots_.size(), 0);
    for (std::uint32_t s : free_) {
        if (s >= slots_.size() || on_free_list[s] != 0 || slots_[s].allocated) return false;
        on_free_list[s] = 1;
    }
    std::uint32_t live = 0;
    for (std::uint32_t s = 0; s < capacity_; ++s) {
        if (slots_[s].allocated) {
            if (slots_[s].generation == PageHandle::kInvalidGeneration || on_free_list[s] != 0) return false;
            ++live;
        } else if (on_free_list[s] == 0) {
            return false;
        }
    }
    return live == allocated_ && releases_ <= allocations_ && allocations_ - releases_ == allocated_;
}

}  // namespace kimkvcache
