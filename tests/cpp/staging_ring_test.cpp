// Ring-order region bookkeeping of the staging ring (ring_regions.h).
//
// Property: a range handed out by reserve() never overlaps a region that is
// still live (not yet retired), and regions retire oldest first.  Replays the
// sequence 768, 256, 512, 768 on a 1024-byte ring (after the wrap the front
// region [768,1024) does not overlap the new [0,768) while the newer [0,512)
// does), then random mixes of large and small requests on several ring
// sizes.
//
// Built by kim-kvcache_amd/build.py; run by tests/test_cpp_contracts.py.
#include "hip/ring_regions.h"

#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

using kimkvcache::RingRegions;

namespace {

int g_failures = 0;

void check(bool ok, char const* what, unsigned long long a = 0, unsigned long long b = 0)
{
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s (%llu, %llu)\n", what, a, b);
        ++g_failures;
    }
}

struct Shadow {
    std::size_t begin;
    std::size_t end;
    std::uint64_t id;
};

// Runs `sizes` through a ring of `capacity` bytes while keeping its own list
// of regions that have not been retired yet.
void replay(std::size_t capacity, std::vector<std::size_t> const& sizes)
{
    RingRegions<std::uint64_t> ring(capacity);
    std::vector<Shadow> live;
    std::uint64_t next_id = 0;
    std::uint64_t next_retire = 0;
    for (std::size_t bytes : sizes) {
        if (bytes == 0 || bytes > ring.maxRequest()) continue;
        std::uint64_t const id = next_id++;
        std::size_t const off = ring.reserve(bytes, id, [&](auto const& r) {
            check(r.tag == next_retire, "regions retire in FIFO order", r.tag, next_retire);
            ++next_retire;
            check(!live.empty() && live.front().id == r.tag, "retired region is the oldest live one", r.tag);
            if (!live.empty()) live.erase(live.begin());
        });
        std::size_t const end = off + ((bytes + 255) & ~std::size_t{255});
        check(off % 256 == 0, "offset is 256-byte aligned", off);
        check(end <= capacity, "range inside the ring", end, capacity);
        for (Shadow const& s : live) {
            check(!(s.begin < end && off < s.end), "new range overlaps a live region", off, s.begin);
        }
        live.push_back(Shadow{off, end, id});
        check(ring.live().size() == live.size(), "live count agrees", ring.live().size(), live.size());
    }
}

}  // namespace

int main()
{
    // The sequence that overwrote a live region when only the front was checked.
    {
        RingRegions<int> ring(1024);
        std::vector<int> retired;
        auto retire = [&](auto const& r) { retired.push_back(r.tag); };
        check(ring.reserve(768, 0, retire) == 0, "first region at 0");
        check(ring.reserve(256, 1, retire) == 768, "second region at 768");
        check(ring.reserve(512, 2, retire) == 0, "third region wraps to 0");
        check(retired.size() == 1 && retired[0] == 0, "wrap retires region 0 only", retired.size());
        check(ring.reserve(768, 3, retire) == 0, "fourth region wraps to 0");
        // [0,768) overlaps region 2 = [0,512); region 1 = [768,1024) is older
        // and retires first.
        check(retired.size() == 3 && retired[1] == 1 && retired[2] == 2, "regions 1 and 2 retire", retired.size());
        check(ring.live().size() == 1 && ring.live().front().tag == 3, "only region 3 is live");
    }
    replay(1024, {768, 256, 512, 768});
    std::mt19937_64 rng(12345);
    for (std::size_t capacity : {std::size_t{1024}, std::size_t{4096}, std::size_t{65536}, std::size_t{8} << 20}) {
        for (int round = 0; round < 200; ++round) {
            std::vector<std::size_t> sizes;
            for (int k = 0; k < 64; ++k) {
                std::uint64_t const pick = rng() % 4;
                std::size_t const big = capacity / 2;
                std::size_t const bytes = pick == 0 ? 1 + rng() % big                 // anything allowed
                                        : pick == 1 ? big - rng() % 512               // near the cap
                                        : pick == 2 ? 1 + rng() % 8192 % big          // small job/item stages
                                                    : 1 + rng() % (capacity / 3);
                sizes.push_back(bytes);
            }
            replay(capacity, sizes);
        }
    }
    if (g_failures != 0) {
        std::fprintf(stderr, "%d failure(s)\n", g_failures);
        return 1;
    }
    std::printf("staging ring: ok\n");
    return 0;
}
