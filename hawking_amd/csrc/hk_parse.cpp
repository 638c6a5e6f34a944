// hk_parse.cpp -- host-only parsing and validation of the on-disk formats
// (hk_parse.h); the loader (hk_container.cpp) binds what these accept.
#include "hk_parse.h"

#include <cstring>
#include <fstream>
#include <sstream>

#include "hk_json.h"

namespace hk {
namespace parse {
namespace {

using json::Value;

const char MAGIC_BINARY[8] = {'H', 'G', 'R', 'A', 'V', 'B', '0', '1'};
const char MAGIC_RESIDUAL[8] = {'H', 'G', 'R', 'A', 'V', 'R', '0', '2'};
const char MAGIC_HGRAVS01[8] = {'H', 'G', 'R', 'A', 'V', 'S', '0', '1'};
const char MAGIC_UNIFORM[8] = {'H', 'G', 'R', 'A', 'V', 'U', '0', '1'};
const char MAGIC_HQ30UQ4[8] = {'H', 'Q', '3', '0', 'U', 'Q', '4', '\0'};
const char MAGIC_HQ30G1B1[8] = {'H', 'Q', '3', '0', 'G', '1', 'B', '1'};
const char MAGIC_CATALOG[8] = {'H', 'Q', '8', '0', 'M', '1', '5', '\0'};
const char* SCHEMA_BINARY = "hawking.gravity.binary_sign_scale.v1";
const char* SCHEMA_RESIDUAL = "hawking.gravity.binary_outlier_residual.v2";
const char* SCHEMA_HGRAVS01 = "hawking.gravity.activation_weighted_svd_low_rank.v1";
const char* SCHEMA_UNIFORM = "hawking.gravity.uniform_group.v1";
const char* HGRAVS01_REPRESENTATION = "activation_weighted_svd_low_rank_q";
const char* CATALOG_SCHEMA = "hawking.ascension.qwen80_mixed_representation_candidate.v1";
constexpr uint32_t CATALOG_VERSION = 1;
constexpr size_t RECORD_SIZE = 128;



uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t rd64(const uint8_t* p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) { return !__builtin_mul_overflow(a, b, out); }
bool add_ok(uint64_t a, uint64_t b, uint64_t* out) { return !__builtin_add_overflow(a, b, out); }
uint64_t div_ceil(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }

Fail bad(const std::string& m) { return Fail{HK_E_INVALID_ARG, m}; }
Fail geom(const std::string& m) { return Fail{HK_E_GEOMETRY, m}; }

// split_gravity_container (q80_mixed_decode.rs:135-147).
bool split(const uint8_t* p, size_t n, const char* magic, const uint8_t** h, size_t* hl, const uint8_t** b, size_t* bl,
           Fail* f) {
    if (n < 12 || std::memcmp(p, magic, 8) != 0) return (*f = bad("gravity container magic mismatch")), false;
    const uint64_t off = 12u + (uint64_t)rd32(p + 8);
    if (off > n) return (*f = geom("gravity container header exceeds payload")), false;
    *h = p + 12;
    *hl = (size_t)(off - 12);
    *b = p + off;
    *bl = n - (size_t)off;
    return true;
}

// header_object / header_str / header_u64 / header_shape / require_header_str
// (q80_mixed_decode.rs:656-737), with the same messages.
bool object(const uint8_t* p, size_t n, const std::string& label, Value* v, Fail* f) {
    std::string e;
    if (!json::parse(p, n, v, &e)) return (*f = bad(label + " header is not JSON: " + e)), false;
    if (v->type != Value::Object) return (*f = bad(label + " header root must be an object")), false;
    return true;
}

bool get_str(const Value& o, const char* key, const std::string& label, std::string* out, Fail* f) {
    const Value* v = o.get(key);
    if (!v || !v->str()) return (*f = bad(label + " missing " + key)), false;
    *out = v->s;
    return true;
}

bool require_str(const Value& o, const char* key, const char* expected, const std::string& label, Fail* f) {
    std::string s;
    if (!get_str(o, key, label, &s, f)) return false;
    if (s != expected) return (*f = bad(label + " " + key + " \"" + s + "\" is not \"" + expected + "\"")), false;
    return true;
}

bool get_u64(const Value& o, const char* key, const std::string& label, uint64_t* out, Fail* f) {
    const Value* v = o.get(key);
    if (!v) return (*f = bad(label + " missing " + key)), false;
    if (v->u64(out)) return true;
    if (v->negative_int()) return (*f = geom(label + " " + key + " is negative")), false;
    return (*f = bad(label + " " + key + " is not an integer")), false;
}

bool get_shape(const Value& o, const char* key, const std::string& label, std::vector<uint64_t>* out, Fail* f) {
    const Value* v = o.get(key);
    if (!v || v->type != Value::Array) return (*f = bad(label + " missing " + key)), false;
    out->clear();
    for (const Value& d : v->arr) {
        uint64_t x;
        if (!d.u64(&x)) return (*f = bad(label + " " + key + " dim is not usize")), false;
        out->push_back(x);
    }
    return true;
}

// matrix_rows_cols (q80_mixed_decode.rs:739-756): [rows, cols]; [len] is
// (len, 1); other ranks stay flat (elements, 1).
bool rows_cols(const std::vector<uint64_t>& shape, uint64_t elements, const std::string& label, uint64_t* rows,
               uint64_t* cols, Fail* f) {
    uint64_t prod = 1;
    for (uint64_t d : shape)
        if (!mul_ok(prod, d, &prod)) return (*f = geom(label + " shape overflows")), false;
    if (prod != elements || elements == 0) return (*f = geom(label + " shape disagrees with elements")), false;
    if (shape.size() == 2) {
        *rows = shape[0];
        *cols = shape[1];
    } else {
        *rows = shape.size() == 1 ? shape[0] : elements;
        *cols = 1;
    }
    return true;
}

std::vector<uint16_t> f16s(const uint8_t* p, size_t count) {
    std::vector<uint16_t> v(count);
    for (size_t i = 0; i < count; ++i) v[i] = rd16(p + 2 * i);
    return v;
}



// uniform_from_body (q80_mixed_decode.rs:788-821): scales f16[groups], then
// the bit-packed codes of groups * group_size elements.
bool uniform_body(uint64_t rows, uint64_t cols, uint64_t bits, uint64_t group, const uint8_t* body, size_t len,
                  const std::string& label, std::vector<uint16_t>* scales, const uint8_t** codes, Fail* f) {
    if (bits < 2 || bits > 8 || group == 0 || rows == 0 || cols == 0)
        return (*f = geom(label + " uniform geometry is invalid")), false;
    uint64_t elements, padded, code_bits;
    if (!mul_ok(rows, cols, &elements)) return (*f = geom(label + " element count overflows")), false;
    const uint64_t groups = div_ceil(elements, group);
    if (!mul_ok(groups, group, &padded) || !mul_ok(padded, bits, &code_bits))
        return (*f = geom(label + " code bytes overflow")), false;
    const uint64_t scale_bytes = groups * 2, code_bytes = div_ceil(code_bits, 8);
    if ((uint64_t)len != scale_bytes + code_bytes)
        return (*f = geom(label + " body " + std::to_string(len) + " != scales " + std::to_string(scale_bytes) +
                           " + codes " + std::to_string(code_bytes))),
               false;
    *scales = f16s(body, (size_t)groups);
    *codes = body + scale_bytes;
    return true;
}

}  // namespace

// parse_binary_group_container (q80_mixed_decode.rs:823-866).
bool parse_binary(const uint8_t* p, size_t n, Body* out, Fail* f) {
    const uint8_t *hb, *body;
    size_t hl, bl;
    Value h;
    const std::string L = "HGRAVB01";
    if (!split(p, n, MAGIC_BINARY, &hb, &hl, &body, &bl, f) || !object(hb, hl, L, &h, f)) return false;
    std::vector<uint64_t> shape;
    uint64_t elements, group, groups, scale_bytes, sign_bytes, rows, cols;
    if (!require_str(h, "schema", SCHEMA_BINARY, L, f) || !get_shape(h, "shape", L, &shape, f) ||
        !get_u64(h, "elements", L, &elements, f) || !get_u64(h, "group_size", L, &group, f) ||
        !get_u64(h, "groups", L, &groups, f) || !get_u64(h, "scale_bytes", L, &scale_bytes, f) ||
        !get_u64(h, "sign_bytes", L, &sign_bytes, f))
        return false;
    uint64_t gbits;
    if (group == 0 || groups != div_ceil(elements, group)) return (*f = geom(L + " group ledger disagrees with elements")), false;
    if (!mul_ok(groups, group, &gbits) || scale_bytes != groups * 2 || sign_bytes != div_ceil(gbits, 8))
        return (*f = geom(L + " scale/sign ledger is invalid")), false;
    if ((uint64_t)bl != scale_bytes + sign_bytes) return (*f = geom(L + " body length disagrees with ledger")), false;
    if (!rows_cols(shape, elements, L, &rows, &cols, f)) return false;
    if (cols % group) return (*f = geom(L + " kernel requires cols to be a multiple of group_size")), false;
    if (groups != rows * (cols / group))
        return (*f = geom(L + " groups are not row-aligned; refuse silent pad reinterpret")), false;
    out->kind = HK_BIN;
    out->group = (int)group;
    out->rows = rows;
    out->cols = cols;
    out->scales = f16s(body, (size_t)groups);
    out->codes = body + scale_bytes;
    out->code_bytes = (size_t)sign_bytes;
    return true;
}

// parse_rice_q1_container (q80_mixed_decode.rs:868-946).
bool parse_residual(const uint8_t* p, size_t n, Body* out, Fail* f) {
    const uint8_t *hb, *body;
    size_t hl, bl;
    Value h;
    const std::string L = "HGRAVR02";
    if (!split(p, n, MAGIC_RESIDUAL, &hb, &hl, &body, &bl, f) || !object(hb, hl, L, &h, f)) return false;
    uint64_t value_bits;
    if (!require_str(h, "schema", SCHEMA_RESIDUAL, L, f) || !require_str(h, "index_mode", "rice", L, f) ||
        !get_u64(h, "value_bits", L, &value_bits, f))
        return false;
    if (value_bits != 1) return (*f = bad(L + " value_bits must be 1 for rice_q1")), false;
    std::vector<uint64_t> shape;
    uint64_t elements, group, groups, scale_bytes, sign_bytes, index_bytes, rscale_bytes, residual_bytes, outliers,
        rice_k, rice_len, first_bytes, rows, cols;
    if (!require_str(h, "value_scale", "rms", L, f) || !get_shape(h, "shape", L, &shape, f) ||
        !get_u64(h, "elements", L, &elements, f) || !get_u64(h, "group_size", L, &group, f) ||
        !get_u64(h, "groups", L, &groups, f) || !get_u64(h, "scale_bytes", L, &scale_bytes, f) ||
        !get_u64(h, "sign_bytes", L, &sign_bytes, f) || !get_u64(h, "index_bytes", L, &index_bytes, f) ||
        !get_u64(h, "residual_scale_bytes", L, &rscale_bytes, f) ||
        !get_u64(h, "residual_bytes", L, &residual_bytes, f) || !get_u64(h, "outlier_count", L, &outliers, f) ||
        !get_u64(h, "rice_k", L, &rice_k, f) || !get_u64(h, "rice_bytes", L, &rice_len, f) ||
        !get_u64(h, "first_index_bytes", L, &first_bytes, f))
        return false;
    if (first_bytes != 4) return (*f = geom(L + " first_index_bytes must be 4")), false;
    if (index_bytes != first_bytes + rice_len) return (*f = geom(L + " index ledger disagrees with rice_bytes")), false;
    if (rscale_bytes != 2) return (*f = geom(L + " rice_q1 requires one fp16 residual scale")), false;
    uint64_t expected = scale_bytes;
    if (!add_ok(expected, sign_bytes, &expected) || !add_ok(expected, index_bytes, &expected) ||
        !add_ok(expected, rscale_bytes, &expected) || !add_ok(expected, residual_bytes, &expected))
        return (*f = geom(L + " body ledger overflows")), false;
    if ((uint64_t)bl != expected) return (*f = geom(L + " body length disagrees with ledger")), false;
    if (!rows_cols(shape, elements, L, &rows, &cols, f)) return false;
    if (group == 0 || cols % group || groups != rows * (cols / group))
        return (*f = geom(L + " binary groups are not row-aligned")), false;
    // the scales must cover the groups and the signs the elements (the
    // reference's slices would fail on a short body at use)
    if (scale_bytes != groups * 2 || sign_bytes < div_ceil(elements, 8) || residual_bytes < div_ceil(outliers, 8))
        return (*f = geom(L + " scale/sign/residual ledger is too short for the shape")), false;
    if (rice_k > 31) return (*f = geom(L + " rice_k must be below 32")), false;
    out->kind = HK_BIN_RICE;
    out->group = (int)group;
    out->rows = rows;
    out->cols = cols;
    out->scales = f16s(body, (size_t)groups);
    size_t c = (size_t)scale_bytes;
    out->codes = body + c;
    out->code_bytes = (size_t)sign_bytes;
    c += (size_t)sign_bytes;
    out->first = rd32(body + c);
    c += 4;
    out->rice = body + c;
    out->rice_bytes = (size_t)rice_len;
    c += (size_t)rice_len;
    out->res_scale = rd16(body + c);
    c += 2;
    out->res_signs = body + c;
    out->outliers = (size_t)outliers;
    out->rice_k = (uint32_t)rice_k;
    return true;
}

// parse_hgravs01_packed_factors (q80_mixed_decode.rs:948-1045).
bool parse_hgravs01(const uint8_t* p, size_t n, Body* out, Fail* f) {
    const uint8_t *hb, *body;
    size_t hl, bl;
    Value h;
    const std::string L = "HGRAVS01";
    if (!split(p, n, MAGIC_HGRAVS01, &hb, &hl, &body, &bl, f) || !object(hb, hl, L, &h, f)) return false;
    if (!require_str(h, "schema", SCHEMA_HGRAVS01, L, f) ||
        !require_str(h, "representation", HGRAVS01_REPRESENTATION, L, f))
        return false;
    const Value* cap = h.get("activation_capture");
    if (!cap || cap->type != Value::Object) return (*f = bad(L + " missing activation_capture")), false;
    if (!require_str(*cap, "fit_kind", "real_routed_activation_capture", L + " activation_capture", f)) return false;
    std::vector<uint64_t> mshape, ls, rs;
    uint64_t rank, bits, group, lbytes, rbytes, lbits, rbits, lgroup, rgroup;
    if (!get_shape(h, "matrix_shape", L, &mshape, f)) return false;
    if (mshape.size() != 2) return (*f = geom(L + " matrix_shape must be rank-2")), false;
    if (!get_u64(h, "rank", L, &rank, f) || !get_u64(h, "factor_bits", L, &bits, f) ||
        !get_u64(h, "factor_group_size", L, &group, f) || !get_u64(h, "left_body_bytes", L, &lbytes, f) ||
        !get_u64(h, "right_body_bytes", L, &rbytes, f))
        return false;
    if (bits > 255) return (*f = geom(L + " factor_bits do not fit u8")), false;
    uint64_t total;
    if (!add_ok(lbytes, rbytes, &total)) return (*f = geom(L + " body ledger overflows")), false;
    if (total != (uint64_t)bl) return (*f = geom(L + " physical body disagrees with factor ledgers")), false;
    const Value* lm = h.get("left");
    const Value* rm = h.get("right");
    if (!lm || lm->type != Value::Object) return (*f = bad(L + " missing left")), false;
    if (!rm || rm->type != Value::Object) return (*f = bad(L + " missing right")), false;
    if (!require_str(*lm, "schema", SCHEMA_UNIFORM, L + " left", f) ||
        !require_str(*rm, "schema", SCHEMA_UNIFORM, L + " right", f) || !get_shape(*lm, "shape", L + " left", &ls, f) ||
        !get_shape(*rm, "shape", L + " right", &rs, f))
        return false;
    if (ls.size() != 2 || rs.size() != 2 || ls[0] != mshape[0] || ls[1] != rank || rs[0] != rank || rs[1] != mshape[1])
        return (*f = geom(L + " factor shapes disagree with matrix_shape/rank")), false;
    if (!get_u64(*lm, "bits", L + " left", &lbits, f) || !get_u64(*rm, "bits", L + " right", &rbits, f) ||
        !get_u64(*lm, "group_size", L + " left", &lgroup, f) || !get_u64(*rm, "group_size", L + " right", &rgroup, f))
        return false;
    if (lbits != bits || rbits != bits || lgroup != group || rgroup != group)
        return (*f = geom(L + " factor bits/group_size disagree with envelope")), false;
    if (!uniform_body(ls[0], ls[1], lbits, lgroup, body, (size_t)lbytes, L + " left", &out->scales, &out->codes, f) ||
        !uniform_body(rs[0], rs[1], rbits, rgroup, body + lbytes, (size_t)rbytes, L + " right", &out->r_scales,
                      &out->r_codes, f))
        return false;
    if (bits != 3 || group != 64)
        return (*f = Fail{HK_E_UNSUPPORTED, L + " factors of " + std::to_string(bits) + " bits / group " +
                                                std::to_string(group) + " (the device kind is 3-bit group 64)"}),
               false;
    out->kind = HK_U3;
    out->group = 64;
    out->rows = ls[0];
    out->cols = ls[1];
    out->r_rows = rs[0];
    out->r_cols = rs[1];
    return true;
}

// parse_uniform_q8_container (q80_mixed_decode.rs:1047-1070).
bool parse_uniform8(const uint8_t* p, size_t n, Body* out, Fail* f) {
    const uint8_t *hb, *body;
    size_t hl, bl;
    Value h;
    const std::string L = "HGRAVU01";
    if (!split(p, n, MAGIC_UNIFORM, &hb, &hl, &body, &bl, f) || !object(hb, hl, L, &h, f)) return false;
    uint64_t bits, group, elements, rows, cols;
    std::vector<uint64_t> shape;
    if (!require_str(h, "schema", SCHEMA_UNIFORM, L, f) || !get_u64(h, "bits", L, &bits, f)) return false;
    if (bits > 255) return (*f = geom(L + " bits do not fit u8")), false;
    if (bits != 8)
        return (*f = geom(L + " bits=" + std::to_string(bits) + " is not the mixed non-expert 8-bit contract")), false;
    if (!get_u64(h, "group_size", L, &group, f)) return false;
    if (group != 64) return (*f = geom(L + " group_size=" + std::to_string(group) + " is not 64")), false;
    if (!get_shape(h, "shape", L, &shape, f) || !get_u64(h, "elements", L, &elements, f) ||
        !rows_cols(shape, elements, L, &rows, &cols, f))
        return false;
    if (!uniform_body(rows, cols, bits, group, body, bl, L, &out->scales, &out->codes, f)) return false;
    out->kind = HK_Q8;
    out->group = 64;
    out->rows = rows;
    out->cols = cols;
    return true;
}

// parse_uniform_q4_header / parse_complete_binary_header: 32-byte header
// {magic[8], u32 version = 1, u32 group_size, u16 rank, u16 0, u64 elements,
// u32 0}, u32 dims[rank], f16 scales[groups], then the codes.
bool parse_hq30(const uint8_t* p, size_t n, Body* out, Fail* f) {
    const bool q4 = n >= 8 && std::memcmp(p, MAGIC_HQ30UQ4, 8) == 0;
    const std::string L = q4 ? "uniform Q4" : "complete binary";
    if (n < 32) return (*f = geom(L + " payload is shorter than its 32-byte header")), false;
    if (!q4 && std::memcmp(p, MAGIC_HQ30G1B1, 8) != 0)
        return (*f = bad("payload magic is neither HQ30UQ4 nor HQ30G1B1")), false;
    const uint32_t version = rd32(p + 8);
    if (version != 1) return (*f = bad(L + " version " + std::to_string(version) + " is unsupported")), false;
    const uint64_t group = rd32(p + 12), rank = rd16(p + 16), elements = rd64(p + 20);
    if (q4 && group != 64 && group != 128)
        return (*f = bad(L + " group_size=" + std::to_string(group) + " must be 64 or 128")), false;
    if (rd16(p + 18) != 0 || rd32(p + 28) != 0) return (*f = bad(L + " reserved header fields must be zero")), false;
    if (!q4 && (group == 0 || group % 8))
        return (*f = bad(L + " group_size=" + std::to_string(group) + " must be a positive multiple of eight")), false;
    if (rank == 0) return (*f = geom(L + " tensor rank must be positive")), false;
    const uint64_t after = 32 + 4 * rank;
    if (after > n) return (*f = geom(L + " is truncated in tensor dimensions")), false;
    std::vector<uint64_t> shape;
    uint64_t derived = 1;
    for (uint64_t d = 0; d < rank; ++d) {
        const uint64_t v = rd32(p + 32 + 4 * d);
        if (v == 0) return (*f = geom(L + " tensor dimensions must be positive")), false;
        if (!mul_ok(derived, v, &derived)) return (*f = geom(L + " tensor element count overflow")), false;
        shape.push_back(v);
    }
    if (elements != derived) return (*f = geom(L + " element count disagrees with shape product")), false;
    const uint64_t groups = div_ceil(elements, group);
    uint64_t code_bytes, end;
    if (!mul_ok(groups, q4 ? group / 2 : group / 8, &code_bytes) || !add_ok(after, groups * 2, &end) ||
        !add_ok(end, code_bytes, &end))
        return (*f = geom(L + " payload byte count overflow")), false;
    if (end != (uint64_t)n)
        return (*f = geom(L + " payload size " + std::to_string(n) + " does not equal fixed-layout expectation " +
                           std::to_string(end))),
               false;
    out->scales = f16s(p + after, (size_t)groups);
    for (size_t g = 0; g < out->scales.size(); ++g)
        if ((out->scales[g] & 0x7C00u) == 0x7C00u)
            return (*f = Fail{HK_E_NONFINITE, L + " scale for group " + std::to_string(g) + " is not finite"}), false;
    // rows_cols of the Q4 tensors (qwen80_uniform_q4_hybrid_decode.rs:266-275)
    if (shape.size() == 2) {
        out->rows = shape[0];
        out->cols = shape[1];
    } else if (shape.size() == 1) {
        out->rows = shape[0];
        out->cols = 1;
    } else {
        return (*f = geom(L + " shape is not a matrix or vector")), false;
    }
    out->kind = q4 ? HK_Q4 : HK_BIN;
    out->group = (int)group;
    out->codes = p + after + groups * 2;
    out->code_bytes = (size_t)code_bytes;
    return true;
}

bool parse_q4_0(const uint8_t* blocks, size_t len, uint32_t rows, uint32_t cols, std::vector<uint16_t>* scales,
                std::vector<uint8_t>* codes, Fail* f) {
    if (rows == 0 || cols == 0 || cols % 32)
        return (*f = geom("q4_0 tensors need rows > 0 and cols % 32 == 0")), false;
    const size_t nb = (size_t)rows * cols / 32;
    if (len != nb * 18)
        return (*f = geom("q4_0 data is " + std::to_string(len) + " bytes, expected " + std::to_string(nb * 18))),
               false;
    scales->resize(nb);
    codes->resize(nb * 16);
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + b * 18;
        (*scales)[b] = rd16(blk);
        uint8_t* c = codes->data() + b * 16;
        for (int i = 0; i < 16; ++i) {
            // canonical byte i holds elements 2i (low) and 2i + 1 (high)
            const int e0 = 2 * i, e1 = 2 * i + 1;
            const uint8_t n0 = e0 < 16 ? (blk[2 + e0] & 0x0F) : (blk[2 + e0 - 16] >> 4);
            const uint8_t n1 = e1 < 16 ? (blk[2 + e1] & 0x0F) : (blk[2 + e1 - 16] >> 4);
            c[i] = (uint8_t)(n0 | (n1 << 4));
        }
    }
    return true;
}

std::string read_file(const std::string& path, bool* ok) {
    std::ifstream in(path, std::ios::binary);
    std::ostringstream ss;
    *ok = (bool)in;
    if (*ok) ss << in.rdbuf();
    return ss.str();
}

bool valid_utf8(const uint8_t* p, size_t n) {
    for (size_t i = 0; i < n;) {
        const uint8_t c = p[i];
        size_t k = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (!k || i + k > n) return false;
        for (size_t j = 1; j < k; ++j)
            if ((p[i + j] & 0xC0) != 0x80) return false;
        i += k;
    }
    return true;
}

// parse_catalog_bytes (qwen80_mixed_catalog.rs:440-555).
std::string parse_catalog(const uint8_t* raw, size_t n, CatalogTable* cat) {
    if (n < 32 || std::memcmp(raw, MAGIC_CATALOG, 8) != 0) return "catalog magic is not HQ80M15";
    const uint32_t version = rd32(raw + 8);
    if (version != CATALOG_VERSION) return "unsupported catalog version " + std::to_string(version);
    const uint64_t n_tensors = rd32(raw + 12), n_segments = rd32(raw + 16), blob = rd32(raw + 24);
    uint64_t c = 32;
    for (uint64_t i = 0; i < n_segments; ++i) {
        if (c + 44 > n) return "segment digest truncated";
        CatalogSegment s;
        s.id = rd16(raw + c);
        const uint64_t name_len = rd16(raw + c + 2);
        s.bytes = rd64(raw + c + 4);
        std::memcpy(s.sha, raw + c + 12, 32);
        c += 44;
        if (c + name_len > n) return "segment name truncated";
        if (!valid_utf8(raw + c, (size_t)name_len)) return "segment name is not utf-8";
        s.filename.assign(reinterpret_cast<const char*>(raw + c), (size_t)name_len);
        c += name_len;
        cat->segments.push_back(std::move(s));
    }
    const uint64_t table_bytes = n_tensors * RECORD_SIZE;
    if (c + table_bytes > n) return "catalog tensor table truncated";
    const uint8_t* table = raw + c;
    c += table_bytes;
    if (c + blob > n) return "catalog name blob truncated";
    const uint8_t* names = raw + c;
    cat->records.resize((size_t)n_tensors);
    cat->names.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        const uint8_t* rec = table + i * RECORD_SIZE;
        hk_catalog_record& r = cat->records[(size_t)i];
        r = hk_catalog_record{};
        const uint64_t name_off = rd32(rec), name_len = rd16(rec + 4);
        r.codec = rec[6];
        r.organ = rec[7];
        r.ndim = rec[8];
        if (r.ndim > 4) return "catalog ndim exceeds 4";
        for (uint32_t d = 0; d < r.ndim; ++d) r.shape[d] = rd32(rec + 12 + 4 * d);
        r.elements = rd64(rec + 28);
        r.segment_id = rd16(rec + 36);
        r.achieved_rank = rd16(rec + 38);
        r.offset = rd64(rec + 40);
        r.nbytes = rd64(rec + 48);
        std::memcpy(r.sha256, rec + 56, 32);
        r.flags = rd32(rec + 88);
        r.n_fit_rows = rd32(rec + 92);
        const uint32_t bpw = rd32(rec + 96);
        std::memcpy(&r.codec_bpw, &bpw, 4);
        if (name_off + name_len > blob) return "tensor name out of blob";
        if (!valid_utf8(names + name_off, (size_t)name_len)) return "tensor name is not utf-8";
        cat->names[(size_t)i].assign(reinterpret_cast<const char*>(names + name_off), (size_t)name_len);
        bool known = false;
        for (const CatalogSegment& s : cat->segments) known |= s.id == r.segment_id;
        if (!known) return "unknown segment_id " + std::to_string(r.segment_id);
        if (!cat->by_name.emplace(cat->names[(size_t)i], (uint32_t)i).second)
            return "catalog contains a duplicate tensor_name";
    }
    for (size_t i = 0; i < cat->records.size(); ++i) cat->records[i].name = cat->names[i].c_str();
    return "";
}

std::string parse_manifest(const uint8_t* raw, size_t n, Manifest* m) {
    Value doc;
    std::string e;
    if (!json::parse(raw, n, &doc, &e)) return "manifest is not JSON: " + e;
    if (doc.type != Value::Object) return "manifest root must be an object";
    const Value* schema = doc.get("schema");
    if (!schema || !schema->str()) return "manifest missing schema";
    if (schema->s != CATALOG_SCHEMA) return "manifest schema \"" + schema->s + "\" is not " + CATALOG_SCHEMA;
    const Value* seal = doc.get("seal_sha256");
    if (!seal || !seal->str()) return "manifest missing seal_sha256";
    m->seal_sha256 = seal->s;
    const Value* ledger = doc.get("complete_physical_bpw_ledger");
    if (!ledger || ledger->type != Value::Object) return "manifest missing complete_physical_bpw_ledger";
    const Value* bpw = ledger->get("complete_physical_bpw");
    if (!bpw || !bpw->f64(&m->complete_physical_bpw)) return "manifest missing complete_physical_bpw";
    const Value* tpb = ledger->get("tensor_payload_bytes");
    if (tpb && !tpb->u64(&m->tensor_payload_bytes)) m->tensor_payload_bytes = 0;
    const Value* cinfo = doc.get("catalog");
    const Value* cpath = cinfo ? cinfo->get("path") : nullptr;
    const Value* csha = cinfo ? cinfo->get("sha256") : nullptr;
    if (!cpath || !cpath->str()) return "manifest missing catalog.path";
    if (!csha || !csha->str()) return "manifest missing catalog.sha256";
    m->catalog_path = cpath->s;
    m->catalog_sha256 = csha->s;
    return "";
}

}  // namespace parse
}  // namespace hk
