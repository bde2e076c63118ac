// SHA-256 of archive ranges (computeWeightDataSha256) against the published
// FIPS 180-2 example digests ("abc", the 448-bit two-block message, one
// million 'a'), a range at an odd offset inside a file, and the refusals of
// a range past the end and of an empty range.
//
// Built by kim-kvcache_amd/build.py; run by tests/test_cpp_contracts.py.
#include "kim-kv/model/weight_manifest.h"

#include <cstdio>
#include <fstream>
#include <string>

using namespace kimkvcache;

namespace {

int g_failures = 0;

std::string digestOf(std::string const& content, std::uint64_t offset, std::uint64_t size)
{
    std::string const path = "/tmp/kimkv_sha256_test.bin";
    {
        std::ofstream out(path, std::ios::binary);
        out.write(content.data(), static_cast<std::streamsize>(content.size()));
    }
    std::string hex;
    WeightManifestStatus const s = computeWeightDataSha256(path, offset, size, hex);
    std::remove(path.c_str());
    return s.ok() ? hex : "error:" + std::string(toString(s.error));
}

void check(std::string const& got, char const* want, char const* what)
{
    if (got != want) {
        std::fprintf(stderr, "FAIL: %s: %s\n", what, got.c_str());
        ++g_failures;
    }
}

}  // namespace

int main()
{
    check(digestOf("abc", 0, 3), "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad", "abc");
    std::string const two = "abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq";
    check(digestOf(two, 0, two.size()), "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
          "448-bit message");
    check(digestOf(std::string(1000000, 'a'), 0, 1000000),
          "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0", "one million 'a'");
    check(digestOf("xx" + two + "yyy", 2, two.size()), "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
          "range inside a file");
    check(digestOf("abc", 1, 3), "error:data_file_mismatch", "range past the end");
    check(digestOf("abc", 0, 0), "error:invalid_argument", "empty range");
    if (g_failures != 0) return 1;
    std::printf("sha256: ok\n");
    return 0;
}
