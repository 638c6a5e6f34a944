// parse_harness.cpp -- drives the loader's host-only parsers
// (hawking_amd/csrc/hk_parse.cpp) under AddressSanitizer and
// UndefinedBehaviorSanitizer: every payload named on the command line is
// parsed whole, at every prefix length (up to 4,096, then in even strides)
// and with single-byte mutations of its first 1,024 bytes, each from a heap
// copy of exactly the bytes in question so that any read past them faults.
// Test infrastructure only (built and run by tests/test_sanitize.py).
//
//   parse_harness KIND FILE [KIND FILE ...]
//   KIND: binary | residual | hgravs01 | uniform8 | hq30 | q4_0:ROWS:COLS |
//         catalog | manifest | selftest-overread | selftest-overflow
// Prints one line per payload: "KIND accepted=0|1 variants=N".
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "hk_parse.h"

using namespace hk::parse;

static bool run(const std::string& kind, const uint8_t* p, size_t n) {
    Body b;
    Fail f{0, ""};
    if (kind == "binary") return parse_binary(p, n, &b, &f);
    if (kind == "residual") return parse_residual(p, n, &b, &f);
    if (kind == "hgravs01") return parse_hgravs01(p, n, &b, &f);
    if (kind == "uniform8") return parse_uniform8(p, n, &b, &f);
    if (kind == "hq30") return parse_hq30(p, n, &b, &f);
    if (kind.rfind("q4_0:", 0) == 0) {
        unsigned rows = 0, cols = 0;
        std::sscanf(kind.c_str() + 5, "%u:%u", &rows, &cols);
        std::vector<uint16_t> s;
        std::vector<uint8_t> c;
        return parse_q4_0(p, n, rows, cols, &s, &c, &f);
    }
    if (kind == "catalog") {
        CatalogTable t;
        return parse_catalog(p, n, &t).empty();
    }
    if (kind == "manifest") {
        Manifest m;
        return parse_manifest(p, n, &m).empty();
    }
    std::fprintf(stderr, "unknown kind %s\n", kind.c_str());
    std::exit(2);
}

// Parse exactly [data, data + n) from a fresh heap block of n bytes.
static bool run_copy(const std::string& kind, const std::vector<uint8_t>& v, size_t n) {
    uint8_t* q = static_cast<uint8_t*>(std::malloc(n ? n : 1));
    if (n) std::memcpy(q, v.data(), n);
    const bool ok = run(kind, n ? q : q + 1, n);  // an empty payload points at the block's end
    std::free(q);
    return ok;
}

int main(int argc, char** argv) {
    if (argc < 3 || argc % 2 == 0) {
        std::fprintf(stderr, "usage: parse_harness KIND FILE [KIND FILE ...]\n");
        return 2;
    }
    for (int a = 1; a + 1 < argc; a += 2) {
        const std::string kind = argv[a];
        if (kind == "selftest-overread") {  // a planted heap over-read (FILE = the block size): ASan must stop here
            const size_t sz = (size_t)std::atoi(argv[a + 1]);
            uint8_t* q = static_cast<uint8_t*>(std::malloc(sz));
            std::memset(q, 0, sz);
            volatile uint8_t x = q[sz];
            std::printf("not stopped %d\n", (int)x);
            std::free(q);
            continue;
        }
        if (kind == "selftest-overflow") {  // a planted signed overflow: UBSan must stop here
            volatile int x = std::atoi(argv[a + 1]);
            std::printf("not stopped %d\n", x + 2147483647);
            continue;
        }
        std::ifstream in(argv[a + 1], std::ios::binary);
        std::vector<uint8_t> v((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
        const size_t n = v.size();
        const bool accepted = run_copy(kind, v, n);
        size_t variants = 1;
        const size_t stride = n > 4096 ? n / 4096 : 1;
        for (size_t m = 0; m < n; m += (m < 4096 ? 1 : stride), ++variants) run_copy(kind, v, m);
        const uint8_t vals[] = {0x00, 0xFF, 0x39, 0x80};
        for (size_t i = 0; i < n && i < 1024; ++i) {
            const uint8_t keep = v[i];
            for (uint8_t x : vals) {
                if (x == keep) continue;
                v[i] = x;
                run_copy(kind, v, n);
                ++variants;
            }
            v[i] = keep;
        }
        std::printf("%s accepted=%d variants=%zu\n", kind.c_str(), accepted ? 1 : 0, variants);
    }
    return 0;
}
