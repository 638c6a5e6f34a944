// hk_parse.h -- host-only parsing and validation of the on-disk formats the
// loader reads (no device code, no HIP headers, so the same source also
// builds into the sanitizer harness, tests/sanitize/parse_harness.cpp):
//
//   * HGRAV* containers: 8-byte magic, u32 little-endian JSON header length,
//     JSON header, body (split_gravity_container and the parse_* functions,
//     model/qwen_complete_binary/q80_mixed_decode.rs:135-147,823-1070).
//   * HQ30UQ4 / HQ30G1B1: 32-byte headers, u32 dimensions, f16 scales, codes
//     (parse_uniform_q4_header, uniform_q4.rs:57-150;
//     parse_complete_binary_header, qwen_complete_binary/mod.rs:137-233).
//   * HQ80M15 catalog bytes and its manifest JSON
//     (qwen80_mixed_catalog.rs:20-33,176-555).
//
// Every function reads only the bytes it is given and reports a failure as a
// status code plus the reference's message.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/hawking_hip.h"

namespace hk {
namespace parse {

// A parse failure: the status code and the reference's message.
struct Fail {
    int code;
    std::string msg;
};

// A canonical body bound to organs (the library copies it during the upload).
struct Body {
    int kind = -1;  // HK_BIN, HK_Q8, HK_U3 (pair), HK_Q4, HK_BIN_RICE
    int group = 0;
    uint64_t rows = 0, cols = 0;
    std::vector<uint16_t> scales;
    const uint8_t* codes = nullptr;
    size_t code_bytes = 0;
    // HGRAVS01 right factor
    uint64_t r_rows = 0, r_cols = 0;
    std::vector<uint16_t> r_scales;
    const uint8_t* r_codes = nullptr;
    // HGRAVR02
    uint32_t first = 0, rice_k = 0;
    const uint8_t* rice = nullptr;
    size_t rice_bytes = 0, outliers = 0;
    uint16_t res_scale = 0;
    const uint8_t* res_signs = nullptr;
};

// By the catalog's codec id (MixedPackedTensor::from_codec_payload,
// q80_mixed_decode.rs:1336-1347).
bool parse_binary(const uint8_t* p, size_t n, Body* out, Fail* f);
bool parse_residual(const uint8_t* p, size_t n, Body* out, Fail* f);
bool parse_hgravs01(const uint8_t* p, size_t n, Body* out, Fail* f);
bool parse_uniform8(const uint8_t* p, size_t n, Body* out, Fail* f);
// HQ30UQ4 (uniform Q4) or HQ30G1B1 (complete binary), by magic.
bool parse_hq30(const uint8_t* p, size_t n, Body* out, Fail* f);

// GGUF Q4_0 (dequant_q4_0, quant.rs:473-498): rows*cols/32 blocks of 18
// bytes {f16 d; u8 qs[16]}, element j < 16 in the low nibble of qs[j] and
// j >= 16 in the high nibble of qs[j - 16], reordered into the canonical
// Q4 group-32 body (scale per block; byte i holds elements 2i low, 2i + 1 high).
bool parse_q4_0(const uint8_t* blocks, size_t len, uint32_t rows, uint32_t cols, std::vector<uint16_t>* scales,
                std::vector<uint8_t>* codes, Fail* f);

std::string read_file(const std::string& path, bool* ok);
bool valid_utf8(const uint8_t* p, size_t n);

// The HQ80M15 catalog: segment table, 128-byte tensor records, name blob.
struct CatalogSegment {
    uint16_t id = 0;
    std::string filename;
    uint64_t bytes = 0;
    uint8_t sha[32] = {};
};
struct CatalogTable {
    std::vector<CatalogSegment> segments;
    std::vector<hk_catalog_record> records;
    std::vector<std::string> names;  // records[i].name points into names[i]
    std::map<std::string, uint32_t> by_name;
};
// parse_catalog_bytes (qwen80_mixed_catalog.rs:440-555); "" on success, else
// the reason.
std::string parse_catalog(const uint8_t* raw, size_t n, CatalogTable* cat);

// The manifest JSON's fields the catalog needs (schema and seal checked,
// catalog path and SHA-256, the bpw ledger); "" on success, else the reason.
struct Manifest {
    std::string seal_sha256, catalog_path, catalog_sha256;
    double complete_physical_bpw = 0.0;
    uint64_t tensor_payload_bytes = 0;
};
std::string parse_manifest(const uint8_t* raw, size_t n, Manifest* m);

}  // namespace parse
}  // namespace hk
