// Region bookkeeping of the pinned staging ring, free of device calls so it
// can be exercised on the CPU.
//
// Regions are handed out in ring order: a request that does not fit between
// the head and the end of the ring starts again at offset 0.  Before a new
// range is returned, every live region that overlaps it must be retired
// (its consumer has finished).  Regions retire in FIFO order, so the ring
// retires the oldest regions up to and including the NEWEST one that
// overlaps the new range; after a wrap that can be a region several places
// behind the front (the front may be an older region at the end of the ring
// that the new range does not touch).
#pragma once

#include <cstddef>
#include <deque>

namespace kimkvcache {

template <typename Tag>
class RingRegions final {
public:
    struct Region {
        std::size_t begin;
        std::size_t end;
        Tag tag;
    };

    static constexpr std::size_t kAlignment = 256;

    explicit RingRegions(std::size_t size) noexcept : size_(size) {}

    [[nodiscard]] std::size_t capacity() const noexcept { return size_; }
    [[nodiscard]] std::deque<Region>& live() noexcept { return live_; }
    [[nodiscard]] std::deque<Region> const& live() const noexcept { return live_; }

    // Largest request reserve() accepts.
    [[nodiscard]] std::size_t maxRequest() const noexcept { return size_ / 2; }

    // Returns the offset of a range of `bytes` (rounded up to kAlignment) and
    // records it as live with `tag`.  `retire(region)` is called for every
    // region that must be complete before the range is reused, oldest first,
    // and the region is dropped right after.  Callers check maxRequest().
    template <typename Retire>
    std::size_t reserve(std::size_t bytes, Tag tag, Retire&& retire)
    {
        bytes = (bytes + kAlignment - 1) & ~(kAlignment - 1);
        std::size_t begin = head_;
        if (begin + bytes > size_) begin = 0;
        std::size_t const end = begin + bytes;
        std::size_t drop = 0;
        for (std::size_t i = live_.size(); i-- > 0;) {
            Region const& r = live_[i];
            if (r.begin < end && begin < r.end) {
                drop = i + 1;
                break;
            }
        }
        for (std::size_t i = 0; i < drop; ++i) {
            retire(live_.front());
            live_.pop_front();
        }
        live_.push_back(Region{begin, end, tag});
        head_ = end;
        return begin;
    }

private:
    std::size_t size_;
    std::size_t head_{0};
    std::deque<Region> live_;
};

}  // namespace kimkvcache
