// The CPU reference surface (kim-kv/reference/kv_reference.h) against what
// IEEE-754 fixes: every binary16 code decodes and re-encodes to itself, every
// midpoint between neighbouring codes rounds to the even one and anything
// off the midpoint to the nearer one, the overflow threshold is 65520; and
// referenceAttention against a long-double softmax written independently.
//
// Built by kim-kvcache_amd/build.py; run by tests/test_cpp_contracts.py.
#include "kim-kv/kim_kv.h"   // the umbrella header must compile on its own
#include "kim-kv/reference/kv_reference.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

using namespace kimkvcache;

namespace {

int g_failures = 0;

void check(bool ok, char const* what, double a = 0, double b = 0)
{
    if (!ok && g_failures < 20) std::fprintf(stderr, "FAIL: %s (%g, %g)\n", what, a, b);
    g_failures += ok ? 0 : 1;
}

bool isNanCode(std::uint16_t c) { return (c & 0x7C00u) == 0x7C00u && (c & 0x3FFu) != 0; }

void codec()
{
    for (std::uint32_t c = 0; c < 0x10000u; ++c) {
        auto const code = static_cast<std::uint16_t>(c);
        float const f = kvScalarToFloat(code);
        if (isNanCode(code)) {
            check(std::isnan(f), "NaN code decodes to NaN", c);
            check(isNanCode(floatToKvScalar(f)), "NaN re-encodes to NaN", c);
            continue;
        }
        check(floatToKvScalar(f) == code, "decode then encode is the identity", c, f);
    }
    // Positive finite neighbours a < b: the midpoint (exact in float: 12 bits)
    // ties to the even code, points just off it go to the nearer code.
    for (std::uint16_t a = 0; a < 0x7BFFu; ++a) {
        auto const b = static_cast<std::uint16_t>(a + 1);
        double const fa = kvScalarToFloat(a);
        double const fb = kvScalarToFloat(b);
        auto const mid = static_cast<float>((fa + fb) / 2);
        check(static_cast<double>(mid) == (fa + fb) / 2, "midpoint exact in float", fa, fb);
        std::uint16_t const even = (a & 1u) == 0 ? a : b;
        check(floatToKvScalar(mid) == even, "midpoint ties to even", fa, fb);
        check(floatToKvScalar(-mid) == (even | 0x8000u), "negative midpoint ties to even", fa, fb);
        check(floatToKvScalar(std::nextafter(mid, 0.0F)) == a, "below the midpoint rounds down", fa, fb);
        check(floatToKvScalar(std::nextafter(mid, 1e9F)) == b, "above the midpoint rounds up", fa, fb);
    }
    check(floatToKvScalar(65519.998F) == 0x7BFFu, "just below 65520 is the largest finite");
    check(floatToKvScalar(65520.0F) == 0x7C00u, "65520 ties to infinity (even)");
    check(floatToKvScalar(1e30F) == 0x7C00u && floatToKvScalar(-1e30F) == 0xFC00u, "overflow to infinity");
    check(floatToKvScalar(std::ldexp(1.0F, -25)) == 0, "2^-25 ties to zero");
    check(floatToKvScalar(std::nextafter(std::ldexp(1.0F, -25), 1.0F)) == 1, "just above 2^-25 is the least subnormal");
    check(floatToKvScalar(1e-30F) == 0 && floatToKvScalar(-1e-30F) == 0x8000u, "underflow keeps the sign");
}

void attention()
{
    std::mt19937 rng(7);
    std::uniform_real_distribution<float> u(-2.0F, 2.0F);
    for (KvLayout layout : {KvLayout{1, 1, 2}, KvLayout{2, 3, 8}, KvLayout{3, 2, 64}}) {
        for (std::uint32_t T : {1u, 2u, 17u, 130u}) {
            std::size_t n = 0;
            check(layout.elementsForTokens(T, n), "layout size");
            std::vector<KvScalar> kv(n);
            for (auto& x : kv) x = floatToKvScalar(u(rng));
            std::size_t const rows = static_cast<std::size_t>(layout.layer_count) * layout.kv_head_count;
            std::size_t const D = layout.head_dimension;
            std::vector<float> q(rows * D);
            for (auto& x : q) x = u(rng);
            std::vector<float> out;
            check(referenceAttention(layout, kv, T, q, out), "valid attention accepted");
            check(out.size() == rows * D, "output size", static_cast<double>(out.size()));
            for (std::uint32_t l = 0; l < layout.layer_count; ++l) {
                for (std::uint32_t h = 0; h < layout.kv_head_count; ++h) {
                    std::size_t const r = static_cast<std::size_t>(l) * layout.kv_head_count + h;
                    std::vector<long double> logit(T);
                    long double top = -1e300L;
                    for (std::uint32_t t = 0; t < T; ++t) {
                        long double dot = 0;
                        for (std::size_t d = 0; d < D; ++d) {
                            dot += static_cast<long double>(q[r * D + d])
                                * kvScalarToFloat(kv[layout.offset(l, KvComponent::Key, t, h, d, T)]);
                        }
                        logit[t] = dot / std::sqrt(static_cast<long double>(D));
                        top = std::max(top, logit[t]);
                    }
                    long double z = 0;
                    for (std::uint32_t t = 0; t < T; ++t) z += std::exp(logit[t] - top);
                    for (std::size_t d = 0; d < D; ++d) {
                        long double want = 0;
                        for (std::uint32_t t = 0; t < T; ++t) {
                            want += std::exp(logit[t] - top) / z
                                * kvScalarToFloat(kv[layout.offset(l, KvComponent::Value, t, h, d, T)]);
                        }
                        double const got = out[r * D + d];
                        check(std::fabs(got - static_cast<double>(want)) <= 2e-5 * (1 + std::fabs(static_cast<double>(want))),
                              "attention matches the long-double softmax", got, static_cast<double>(want));
                    }
                }
            }
        }
    }
    KvLayout const layout{1, 1, 2};
    std::vector<KvScalar> kv(8, 0);
    std::vector<float> out{42.0F};
    check(!referenceAttention(layout, kv, 0, {1.0F, 0.0F}, out) && out.size() == 1, "zero tokens rejected");
    check(!referenceAttention(layout, kv, 2, {1.0F}, out) && out[0] == 42.0F, "query size rejected");
    check(!referenceAttention(layout, kv, 3, {1.0F, 0.0F}, out), "kv size rejected");
}

}  // namespace

int main()
{
    codec();
    attention();
    if (g_failures != 0) {
        std::fprintf(stderr, "%d failure(s)\n", g_failures);
        return 1;
    }
    std::printf("kv reference: ok\n");
    return 0;
}
