// hk_container.cpp -- the loader: on-disk organ containers and the mixed
// catalog, parsed and validated on the host the way the reference's loaders
// do (hk_parse.cpp), then bound through the organ uploads (canonical bodies
// are uploaded and repacked once, as for any other organ).
//
//   * HGRAV* containers by the catalog's codec id
//     (MixedPackedTensor::from_codec_payload, q80_mixed_decode.rs:1336-1347).
//   * HQ30UQ4 / HQ30G1B1 payloads with their 32-byte headers.
//   * HQ80M15 catalog: manifest JSON -> catalog file (SHA-256 checked) ->
//     segments table, 128-byte tensor records, name blob; payload windows of
//     memory-mapped segment files, SHA-256 checked on first use
//     (qwen80_mixed_catalog.rs:20-33,176-555).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <memory>
#include <set>

#include "hk_internal.h"
#include "hk_parse.h"
#include "hk_sha256.h"

namespace hk {
namespace {

using parse::Body;
using parse::Fail;

// Upload a parsed body; HGRAVS01 gives two organs.
int bind(hk_ctx* ctx, const Body& b, hk_stream stream, hk_organ** out, hk_organ** right) {
    if (b.rows > 0xFFFFFFFFull || b.cols > 0xFFFFFFFFull || b.r_rows > 0xFFFFFFFFull || b.r_cols > 0xFFFFFFFFull)
        return set_error(ctx, HK_E_GEOMETRY, "tensor dimensions exceed u32");
    if (b.kind == HK_BIN_RICE) {
        hk_rice_q1 s{};
        s.rows = (uint32_t)b.rows;
        s.cols = (uint32_t)b.cols;
        s.bin_scales = b.scales.data();
        s.bin_signs = b.codes;
        s.first_index = b.first;
        s.rice_k = b.rice_k;
        s.rice = b.rice_bytes ? b.rice : nullptr;
        s.rice_bytes = b.rice_bytes;
        s.outlier_count = b.outliers;
        s.residual_scale_f16 = b.res_scale;
        s.residual_signs = b.res_signs;
        if (b.group != 128) return set_error(ctx, HK_E_UNSUPPORTED, "HGRAVR02 binary base must use group_size 128");
        return hk_organ_upload_rice(ctx, &s, stream, out);
    }
    hk_organ_src s{};
    s.kind = b.kind;
    s.group = b.group;
    s.rows = (uint32_t)b.rows;
    s.cols = (uint32_t)b.cols;
    s.scales = b.scales.data();
    s.codes = b.codes;
    int rc = hk_organ_upload(ctx, &s, stream, out);
    if (rc || b.kind != HK_U3) return rc;
    hk_organ_src r{};
    r.kind = HK_U3;
    r.group = 64;
    r.rows = (uint32_t)b.r_rows;
    r.cols = (uint32_t)b.r_cols;
    r.scales = b.r_scales.data();
    r.codes = b.r_codes;
    rc = hk_organ_upload(ctx, &r, stream, right);
    if (rc) {
        const std::string msg = ctx->last_error;
        (void)hk_organ_free(ctx, *out);
        *out = nullptr;
        return set_error(ctx, rc, "HGRAVS01 right factor: " + msg);
    }
    return HK_OK;
}

}  // namespace
}  // namespace hk

using namespace hk;

// ====================================================================== containers

extern "C" int hk_organ_from_container(hk_ctx* ctx, int32_t codec, const uint8_t* payload, size_t len,
                                       hk_stream stream, hk_organ** out, hk_organ** right) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (right) *right = nullptr;
    if (!payload && len) return set_error(ctx, HK_E_INVALID_ARG, "hk_organ_from_container: NULL payload");
    Body b;
    Fail f{HK_OK, ""};
    bool ok;
    switch (codec) {
    case HK_CODEC_BINARY: ok = parse::parse_binary(payload, len, &b, &f); break;
    case HK_CODEC_RESIDUAL: ok = parse::parse_residual(payload, len, &b, &f); break;
    case HK_CODEC_HGRAVS01: ok = parse::parse_hgravs01(payload, len, &b, &f); break;
    case HK_CODEC_UNIFORM8: ok = parse::parse_uniform8(payload, len, &b, &f); break;
    default: return set_error(ctx, HK_E_INVALID_ARG, "unknown mixed codec " + std::to_string(codec));
    }
    if (!ok) return set_error(ctx, f.code, f.msg);
    if (b.kind == HK_U3 && !right)
        return set_error(ctx, HK_E_INVALID_ARG, "HGRAVS01 binds two organs: pass `right`");
    return bind(ctx, b, stream, out, right);
}

extern "C" int hk_organ_from_hq30(hk_ctx* ctx, const uint8_t* payload, size_t len, hk_stream stream, hk_organ** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (!payload) return set_error(ctx, HK_E_INVALID_ARG, "hk_organ_from_hq30: NULL payload");
    Body b;
    Fail f{HK_OK, ""};
    if (!parse::parse_hq30(payload, len, &b, &f)) return set_error(ctx, f.code, f.msg);
    return bind(ctx, b, stream, out, nullptr);
}

// GGUF Q4_0 blocks (dequant_q4_0, quant.rs:473-498): per 32 elements
// {f16 d; u8 qs[16]}, element j < 16 in the low nibble of qs[j], element
// j >= 16 in the high nibble of qs[j - 16].  The canonical Q4 group-32 body
// keeps d as the group's scale and the nibbles unchanged, paired (2i, 2i+1)
// per byte, so the bound organ decodes to the same (nibble - 8) * d.
extern "C" int hk_organ_from_q4_0(hk_ctx* ctx, const uint8_t* blocks, size_t len, uint32_t rows, uint32_t cols,
                                  hk_stream stream, hk_organ** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (!blocks) return set_error(ctx, HK_E_INVALID_ARG, "hk_organ_from_q4_0: NULL blocks");
    std::vector<uint16_t> scales;
    std::vector<uint8_t> codes;
    Fail f{HK_OK, ""};
    if (!parse::parse_q4_0(blocks, len, rows, cols, &scales, &codes, &f)) return set_error(ctx, f.code, f.msg);
    hk_organ_src src{};
    src.kind = HK_Q4;
    src.group = 32;
    src.rows = rows;
    src.cols = cols;
    src.scales = scales.data();
    src.codes = codes.data();
    return hk_organ_upload(ctx, &src, stream, out);
}

// ====================================================================== catalog

struct hk_catalog {
    std::string root;
    std::string seal_sha256;
    double complete_physical_bpw = 0.0;
    uint64_t tensor_payload_bytes = 0;
    hk::parse::CatalogTable t;
    // per segment (t.segments order): its file, mapped on first use
    struct Map {
        std::string path;
        const uint8_t* p = nullptr;
        size_t len = 0;
    };
    std::vector<Map> maps;
    std::set<uint32_t> verified;

    ~hk_catalog() {
        for (Map& m : maps)
            if (m.p) munmap(const_cast<uint8_t*>(m.p), m.len);
    }
};

extern "C" int hk_catalog_open(hk_ctx* ctx, const char* manifest_path, hk_catalog** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (!manifest_path) return set_error(ctx, HK_E_INVALID_ARG, "hk_catalog_open: NULL path");
    const std::string mpath(manifest_path);
    const std::string pre = "qwen80 mixed catalog: ";
    bool ok;
    const std::string raw = parse::read_file(mpath, &ok);
    if (!ok) return set_error(ctx, HK_E_INVALID_ARG, pre + "cannot read " + mpath);
    parse::Manifest man;
    std::string e = parse::parse_manifest(reinterpret_cast<const uint8_t*>(raw.data()), raw.size(), &man);
    if (!e.empty()) return set_error(ctx, HK_E_INVALID_ARG, pre + e);
    std::unique_ptr<hk_catalog> cat(new hk_catalog());
    const size_t slash = mpath.find_last_of('/');
    cat->root = slash == std::string::npos ? "." : mpath.substr(0, slash);
    cat->seal_sha256 = man.seal_sha256;
    cat->complete_physical_bpw = man.complete_physical_bpw;
    cat->tensor_payload_bytes = man.tensor_payload_bytes;
    const std::string catalog_path =
        (!man.catalog_path.empty() && man.catalog_path[0] == '/') ? man.catalog_path : cat->root + "/" + man.catalog_path;
    const std::string bytes = parse::read_file(catalog_path, &ok);
    if (!ok) return set_error(ctx, HK_E_INVALID_ARG, pre + "cannot read catalog " + catalog_path);
    uint8_t d[32];
    Sha256::of(reinterpret_cast<const uint8_t*>(bytes.data()), bytes.size(), d);
    if (Sha256::hex(d) != man.catalog_sha256)
        return set_error(ctx, HK_E_INVALID_ARG,
                         pre + "catalog sha256 " + Sha256::hex(d) + " != manifest " + man.catalog_sha256);
    e = parse::parse_catalog(reinterpret_cast<const uint8_t*>(bytes.data()), bytes.size(), &cat->t);
    if (!e.empty()) return set_error(ctx, HK_E_GEOMETRY, pre + e);
    for (const parse::CatalogSegment& s : cat->t.segments)
        cat->maps.push_back(hk_catalog::Map{cat->root + "/segments/" + s.filename, nullptr, 0});
    *out = cat.release();
    return HK_OK;
}

extern "C" int hk_catalog_close(hk_catalog* cat) {
    delete cat;
    return HK_OK;
}

extern "C" int hk_catalog_info(const hk_catalog* cat, uint32_t* n_tensors, uint32_t* n_segments,
                               double* complete_physical_bpw, uint64_t* tensor_payload_bytes) {
    if (!cat) return HK_E_INVALID_ARG;
    if (n_tensors) *n_tensors = (uint32_t)cat->t.records.size();
    if (n_segments) *n_segments = (uint32_t)cat->t.segments.size();
    if (complete_physical_bpw) *complete_physical_bpw = cat->complete_physical_bpw;
    if (tensor_payload_bytes) *tensor_payload_bytes = cat->tensor_payload_bytes;
    return HK_OK;
}

extern "C" int hk_catalog_record_at(const hk_catalog* cat, uint32_t index, hk_catalog_record* out) {
    if (!cat || !out || index >= cat->t.records.size()) return HK_E_INVALID_ARG;
    *out = cat->t.records[index];
    return HK_OK;
}

extern "C" int hk_catalog_find(hk_ctx* ctx, const hk_catalog* cat, const char* name, hk_catalog_record* out) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!cat || !name || !out) return set_error(ctx, HK_E_INVALID_ARG, "hk_catalog_find: NULL argument");
    const auto it = cat->t.by_name.find(name);
    if (it == cat->t.by_name.end())
        return set_error(ctx, HK_E_INVALID_ARG, std::string("qwen80 mixed catalog: missing tensor \"") + name + "\"");
    *out = cat->t.records[it->second];
    return HK_OK;
}

// payload_view (qwen80_mixed_catalog.rs:376-438): the record's window of its
// mapped segment, its SHA-256 checked the first time unless verify is 0.
extern "C" int hk_catalog_payload(hk_ctx* ctx, hk_catalog* cat, const char* name, int verify_sha256,
                                  const uint8_t** data, size_t* len) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!cat || !name || !data || !len) return set_error(ctx, HK_E_INVALID_ARG, "hk_catalog_payload: NULL argument");
    const std::string pre = "qwen80 mixed catalog: ";
    const auto it = cat->t.by_name.find(name);
    if (it == cat->t.by_name.end()) return set_error(ctx, HK_E_INVALID_ARG, pre + "missing tensor \"" + name + "\"");
    const hk_catalog_record& r = cat->t.records[it->second];
    hk_catalog::Map* seg = nullptr;  // parse_catalog admits only records of a listed segment
    for (size_t i = 0; i < cat->t.segments.size(); ++i)
        if (cat->t.segments[i].id == r.segment_id) seg = &cat->maps[i];
    if (!seg->p) {
        const int fd = open(seg->path.c_str(), O_RDONLY);
        if (fd < 0) return set_error(ctx, HK_E_INVALID_ARG, pre + "cannot open segment " + seg->path);
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) {
            close(fd);
            return set_error(ctx, HK_E_INVALID_ARG, pre + "cannot stat segment " + seg->path);
        }
        void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (m == MAP_FAILED) return set_error(ctx, HK_E_INVALID_ARG, pre + "cannot mmap segment " + seg->path);
        seg->p = static_cast<const uint8_t*>(m);
        seg->len = (size_t)st.st_size;
    }
    uint64_t end;
    if (__builtin_add_overflow(r.offset, r.nbytes, &end) || end > seg->len)
        return set_error(ctx, HK_E_GEOMETRY, pre + "\"" + name + "\" range exceeds its segment");
    const uint8_t* p = seg->p + r.offset;
    if (verify_sha256 && !cat->verified.count(it->second)) {
        uint8_t d[32];
        Sha256::of(p, (size_t)r.nbytes, d);
        if (std::memcmp(d, r.sha256, 32) != 0)
            return set_error(ctx, HK_E_GEOMETRY, pre + "\"" + name + "\" payload sha256 " + Sha256::hex(d) +
                                                     " != catalog " + Sha256::hex(r.sha256));
        cat->verified.insert(it->second);
    }
    *data = p;
    *len = (size_t)r.nbytes;
    return HK_OK;
}

// load_packed (qwen80_mixed_catalog.rs:432-436): the payload through
// from_codec_payload's codec dispatch, bound to organs.
extern "C" int hk_catalog_load(hk_ctx* ctx, hk_catalog* cat, const char* name, int verify_sha256, hk_stream stream,
                               hk_organ** out, hk_organ** right) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (right) *right = nullptr;
    const uint8_t* p = nullptr;
    size_t n = 0;
    int rc = hk_catalog_payload(ctx, cat, name, verify_sha256, &p, &n);
    if (rc) return rc;
    hk_catalog_record r;
    (void)hk_catalog_find(ctx, cat, name, &r);
    return hk_organ_from_container(ctx, (int32_t)r.codec, p, n, stream, out, right);
}
