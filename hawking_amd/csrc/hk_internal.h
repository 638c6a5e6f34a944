// hk_internal.h -- shared host/device definitions of the HIP library.
//
// Device-side layouts (all little-endian, all device memory owned by the
// library unless a caller passes its own pointers):
//
//   Q4 organ   (kind HK_Q4, group G in {32,64,128}): canonical SoA, as the
//              reference's HQ30UQ4 body: f16 scales[rows*cols/G] then
//              u8 codes[rows*cols/2]; element e -> byte e/2, even e in the
//              low nibble, value (nibble-8)*scale[e/G].
//   BIN organ  (kind HK_BIN, group 128): HGRAVB01 body: f16 scales[rows*cols/128]
//              then u8 signs[rows*cols/8], bit (e&7) of byte e>>3, 1 -> +scale.
//   MIXED      (kind HK_MIXED): tags bitmap (1 = binary, LSB-first over flat
//              128-groups) + binary section (f16 scale, 16 B signs per group)
//              + Q2 section (2 f16 scales, 32 B 2-bit codes per group), plus two
//              u32[rows+1] prefix tables giving each row's first binary and Q2
//              group, so a row is addressable without a scan.
//   F32 dense  (kind HK_F32): row-major f32[rows*cols].
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/hawking_hip.h"

namespace hk {

// ------------------------------------------------------------------ device organ views

// An organ in the canonical (reference) byte layout described above; the
// load-time repack reads it, and the MoE model stores experts in it.
struct CanonView {
    int32_t kind;
    int32_t group;
    uint32_t rows;
    uint32_t cols;
    const uint16_t* scales;     // Q4 / BIN scales, MIXED binary scales
    const uint8_t* codes;       // Q4 codes, BIN signs, MIXED binary signs
    const uint8_t* tags;        // MIXED
    const uint16_t* q2_scales;  // MIXED
    const uint8_t* q2_codes;    // MIXED
    const uint32_t* row_bin;    // MIXED, [rows+1]
    const uint32_t* row_q2;     // MIXED, [rows+1]
    const float* dense;         // F32
};

// An organ in the wavefront-tiled layout (hk_tile.h) the GEMV kernels read.
struct OrganView {
    int32_t kind;
    int32_t group;
    uint32_t rows;
    uint32_t cols;
    uint32_t n_tiles;           // ceil(rows / 16)
    uint32_t steps;             // 1 KiB wave loads per tile (U3: 768 B)
    uint32_t tail_q;            // U3: column slots stored in the last step (1..4)
    uint32_t reserved;
    const uint8_t* data;        // signs / codes / mixed items
    const uint16_t* scales;
    const uint4* hdr;           // MIXED per-(tile, step) headers
    const float* dense;         // F32 (row-major, not tiled)
};

// ------------------------------------------------------------------ device helpers

// Loads through a global-address-space pointer.  Pointers read out of
// descriptor structs are generic to the compiler, which then emits flat loads;
// a flat load counts in both vmcnt and lgkmcnt, so every later LDS wait also
// waits for it and a software prefetch pipeline collapses to depth one.
template <class T>
__device__ __forceinline__ T ldg(const T* p) {
    return *(const __attribute__((address_space(1))) T*)(p);
}
typedef unsigned int hk_u32x4 __attribute__((ext_vector_type(4)));
typedef float hk_f32x4 __attribute__((ext_vector_type(4)));
// *(base + byte_off bytes): a 32-bit byte offset from a uniform base takes
// the scalar-base load form (an element index scaled in 64 bits would cost a
// 64-bit address per lane).
template <class T>
__device__ __forceinline__ T ldg_at(const T* base, uint32_t byte_off) {
    return ldg(reinterpret_cast<const T*>(reinterpret_cast<const uint8_t*>(base) + byte_off));
}
__device__ __forceinline__ uint4 ldg(const uint4* p) {
    const hk_u32x4 v = *(const __attribute__((address_space(1))) hk_u32x4*)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
typedef unsigned int hk_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ldg(const uint2* p) {
    const hk_u32x2 v = *(const __attribute__((address_space(1))) hk_u32x2*)(p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float4 ldg(const float4* p) {
    const hk_f32x4 v = *(const __attribute__((address_space(1))) hk_f32x4*)(p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// Streaming loads of data read once (weights): the non-temporal hint (the
// load's nt bit) lets HBM deliver 7.1 TB/s to a plain read stream against
// 6.4 TB/s for ordinary loads (4 GiB, 16-byte loads, 4-8k workgroups).
template <class T>
__device__ __forceinline__ T ldg_nt(const T* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) T*)(p));
}
__device__ __forceinline__ uint4 ldg_nt(const uint4* p) {
    const hk_u32x4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) hk_u32x4*)(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg_nt(const uint2* p) {
    const hk_u32x2 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) hk_u32x2*)(p));
    return make_uint2(v.x, v.y);
}
template <class T>
__device__ __forceinline__ T ldg_nt_at(const T* base, uint32_t byte_off) {
    return ldg_nt(reinterpret_cast<const T*>(reinterpret_cast<const uint8_t*>(base) + byte_off));
}

// Copies n16 16-byte pieces from global memory to dst (LDS) with `nthreads`
// threads (this one is `tid`); each thread issues PT loads before its first
// store, so the copy costs about one memory latency per PT * nthreads pieces
// (a load-then-store loop would wait for every load in turn).  The loads are
// unconditional (an index past the end re-reads the last piece), so no branch
// holds them back.
template <int PT>
__device__ __forceinline__ void copy16_to_lds(uint4* dst, const uint4* src, uint32_t n16, uint32_t tid,
                                              uint32_t nthreads) {
    for (uint32_t b = 0; b < n16; b += PT * nthreads) {
        uint4 v[PT];
#pragma unroll
        for (int i = 0; i < PT; ++i) v[i] = ldg(src + min(b + tid + (uint32_t)i * nthreads, n16 - 1u));
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const uint32_t k = b + tid + (uint32_t)i * nthreads;
            if (k < n16) dst[k] = v[i];
        }
    }
}

// Two such copies at once (src0 -> dst0 with n0 pieces, then src1 -> dst1
// with n1) sharing one batch of loads: one latency where two calls of
// copy16_to_lds would take two.
template <int PT>
__device__ __forceinline__ void copy16x2_to_lds(uint4* dst0, const uint4* src0, uint32_t n0, uint4* dst1,
                                                const uint4* src1, uint32_t n1, uint32_t tid, uint32_t nthreads) {
    const uint32_t n = n0 + n1;
    for (uint32_t b = 0; b < n; b += PT * nthreads) {
        uint4 v[PT];
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const uint32_t k = b + tid + (uint32_t)i * nthreads;
            if (k < n) v[i] = ldg(k < n0 ? src0 + k : src1 + (k - n0));
        }
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const uint32_t k = b + tid + (uint32_t)i * nthreads;
            if (k < n0) dst0[k] = v[i];
            else if (k < n) dst1[k - n0] = v[i];
        }
    }
}

// Three such copies at once, every load unconditional (an index past the
// end re-reads the last piece of src2): one latency for all three.
template <int PT>
__device__ __forceinline__ void copy16x3_to_lds(uint4* dst0, const uint4* src0, uint32_t n0, uint4* dst1,
                                                const uint4* src1, uint32_t n1, uint4* dst2, const uint4* src2,
                                                uint32_t n2, uint32_t tid, uint32_t nthreads) {
    const uint32_t n01 = n0 + n1, n = n01 + n2;
    for (uint32_t b = 0; b < n; b += PT * nthreads) {
        uint4 v[PT];
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const uint32_t k = b + tid + (uint32_t)i * nthreads;
            v[i] = ldg(k < n0 ? src0 + k : k < n01 ? src1 + (k - n0) : src2 + min(k - n01, n2 - 1u));
        }
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const uint32_t k = b + tid + (uint32_t)i * nthreads;
            if (k < n0) dst0[k] = v[i];
            else if (k < n01) dst1[k - n0] = v[i];
            else if (k < n) dst2[k - n01] = v[i];
        }
    }
}

// Workgroup -> (organ, part).  Workgroups are dispatched to the 8 XCDs round
// robin by linear id, so ids 8 apart share an XCD and its L2: each run of
// 8 * parts ids covers 8 organs with id % 8 selecting the organ, and all
// parts of an organ (which read the same x) land on one XCD.
// Make a kernel-argument value available here: the argument segment is
// fresh memory at every launch (a full memory round trip), and the compiler
// otherwise loads each field where a branch first needs it, one round trip
// per branch level; a kernel that branches on its arguments names the fields
// its branches read at its top, so all are loaded in one round.  Emits no
// instruction.
template <class V>
__device__ __forceinline__ void arg_here(V v) {
    asm volatile("" ::"s"(v));
}
__device__ __forceinline__ void view_here(const OrganView& o) {
    arg_here(o.data);
    arg_here(o.scales);
    arg_here(o.steps);
    arg_here(o.n_tiles);
    arg_here(o.rows);
    arg_here(o.cols);
}

__device__ __forceinline__ void organ_part(uint32_t L, uint32_t parts, uint32_t n, uint32_t* organ, uint32_t* part) {
    const uint32_t c = L / (8u * parts), r = L % (8u * parts), g = min(8u, n - 8u * c);
    *organ = 8u * c + r % g;
    *part = r / g;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// Wave-wide reductions on the DPP network (VALU lane moves, no LDS round
// trips): an inclusive scan within each 16-lane row (row_shr 1, 2, 4, 8),
// then row_bcast:15 / row_bcast:31 fold the rows into lane 63, which is
// broadcast.  Lanes whose DPP source is outside the row keep the identity.
// All 64 lanes must be active.
constexpr int DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118;
constexpr int DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i32(int identity, int v) {
    return __builtin_amdgcn_update_dpp(identity, v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float identity, float v) {
    return __builtin_bit_cast(float, dpp_i32<CTRL, ROW_MASK>(__builtin_bit_cast(int, identity), __builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float lane63_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Full-wave (64 lanes) sum; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<DPP_ROW_SHR1, 0xF>(0.0f, v);
    v += dpp_f32<DPP_ROW_SHR2, 0xF>(0.0f, v);
    v += dpp_f32<DPP_ROW_SHR4, 0xF>(0.0f, v);
    v += dpp_f32<DPP_ROW_SHR8, 0xF>(0.0f, v);
    v += dpp_f32<DPP_ROW_BCAST15, 0xA>(0.0f, v);
    v += dpp_f32<DPP_ROW_BCAST31, 0xC>(0.0f, v);
    return lane63_f32(v);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<DPP_ROW_SHR1, 0xF>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_SHR2, 0xF>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_SHR4, 0xF>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_SHR8, 0xF>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_BCAST15, 0xA>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_BCAST31, 0xC>(-INFINITY, v));
    return lane63_f32(v);
}

// ------------------------------------------------------------------ host error plumbing

struct Status {
    int code = HK_OK;
    std::string msg;
};

}  // namespace hk

// Context: one per host thread (not thread-safe), bound to one device.
struct hk_ctx {
    int device = 0;
    int last_status = HK_OK;
    std::string last_error;
    // Device word that kernels OR error bits into (read by hk_check_device_status).
    uint32_t* dev_status = nullptr;
    // The packers' non-finite flag (its own 256-byte allocation; the packers
    // synchronise their stream before they return, so calls never overlap).
    uint32_t* pack_flag = nullptr;
    // This device's copy of the no-allocation workspace (a static device
    // array), looked up on the first hk_terminal_greedy_noalloc call.
    uint8_t* noalloc = nullptr;
};

namespace hk {

int set_error(hk_ctx* ctx, int code, const std::string& msg);
int check_hip(hk_ctx* ctx, hipError_t e, const char* what);

// Kernel launchers (defined in the .hip files); all stream-ordered, no sync.
// GEMV over n organs of one kind/shape (descriptor table in device memory).
// Dynamic LDS of the GEMV kernel for a packed organ of `cols` columns (x
// image, quantization window, mixed headers, row outputs), and its cap of
// 64 KB (two workgroups per CU of 160 KB at the widest organs).
size_t gemv_lds_bytes(int kind, uint32_t cols);
constexpr size_t GEMV_LDS_LIMIT = 64 * 1024;
struct ResView;
// The binary GEMV of HGRAVR02 organs with the residual added in its
// epilogue (the bits of launch_gemv_tiled then launch_rice_apply); pieces256
// / pieces512: rice_part_pieces of the organs for 256- and 512-row parts.
// *fused = false (nothing launched) when the launch shape has no fused form.
hipError_t launch_gemv_rice(const OrganView* organs_dev, const ResView* res_dev, uint32_t n, const OrganView& sh,
                            uint32_t pieces256, uint32_t pieces512, const float* x, size_t x_stride, float* y,
                            size_t y_stride, hipStream_t s, bool* fused);
// The read-only bandwidth control (hk_control.hip).
hipError_t launch_stream_control(const void* data, size_t nbytes, float* out, uint32_t workgroups, hipStream_t s);
hipError_t launch_gemv_tiled(const OrganView* organs_dev, uint32_t n, const OrganView& shape,
                             const float* x, size_t x_stride, float* y, size_t y_stride,
                             hipStream_t s);
hipError_t launch_decode_rows(const OrganView& o, uint32_t row0, uint32_t nrows, float* out,
                              hipStream_t s);
// Canonical -> tiled repack of one organ; `scratch` holds >= 8*(n_tiles*steps+1) bytes.
hipError_t launch_repack(const CanonView& src, const OrganView& dst, void* scratch, hipStream_t s);
// The same for n organs of one kind (job table in device memory; mixed jobs
// carry a count array of n_tiles*steps words each).  max_items = the largest
// n_tiles*steps*64 of the jobs.
struct RepackJob {
    CanonView src;
    OrganView dst;
    uint32_t* counts;
};
hipError_t launch_repack_batch(int kind, const RepackJob* jobs_dev, uint32_t n, size_t max_items, hipStream_t s);
// The residual of an HGRAVR02 organ on the device: CSR over its outliers,
// row_ptr[rows + 1] and recs[count] = column << 1 | sign (sign 1 = +scale),
// each row's records in index order and padded to a multiple of 4 with the
// record cols << 1 (a column past the end: adds nothing); count (the padded
// total) is a multiple of 4 and recs is readable to the next multiple of 8.
//
// The fused GEMV reads the same records as byte steps (row_ptr8, recs8,
// count8; rice_step_records): a row's records index a table of three
// entries per column (3c: -p, 3c + 1: +p, 3c + 2: -0; then 8 entries of -0
// past the last column, rice_table3_bytes), each byte the step from the
// previous index (a row starts at -1); a gap wider than one byte steps
// through -0 entries, and rows are padded to 4 bytes with steps onto -0
// entries.  Adding -0 changes no sum, so the totals are the CSR's to the bit.
struct ResView {
    const uint32_t* row_ptr;
    const uint16_t* recs;
    uint32_t rows, cols;
    float scale;
    uint32_t count;
    const uint32_t* row_ptr8;  // [rows + 1], byte offsets into recs8
    const uint8_t* recs8;      // count8 bytes, readable to the next multiple of 16
    uint32_t count8;
};
// status |= 16 if any of the n f16 values is not finite.
hipError_t launch_f16_check(const uint16_t* v, size_t n, uint32_t* status, hipStream_t s);
// Adds the outliers of rows [row0, row0 + nrows) to a decoded base.
hipError_t launch_rice_decode_add(const ResView& v, uint32_t row0, uint32_t nrows, float* out, hipStream_t s);
// y_i += R_i x_i for n residuals of one shape (table in device memory).
// pieces: the most 16-byte record pieces any RICE_APPLY_ROWS-row part of the
// n residuals spans (rice_part_pieces).
constexpr uint32_t RICE_APPLY_ROWS = 512;
// Bytes of the apply's signed product table in LDS: T[2 c + sign] =
// (sign ? scale : -scale) * x[c] for c < cols, T[2 cols] = -0 (the padding
// records' entry), 16-byte aligned.
__host__ __device__ inline size_t rice_table_bytes(uint32_t cols) { return ((size_t)cols * 8u + 8u + 15u) & ~(size_t)15; }
uint32_t rice_part_pieces(const uint32_t* row_ptr, uint32_t rows, uint32_t part_rows);
// The byte-step records' table: 3 cols + 8 floats, 16-byte aligned.
__host__ __device__ inline size_t rice_table3_bytes(uint32_t cols) { return ((size_t)cols * 12u + 32u + 15u) & ~(size_t)15; }
// The most 16-byte pieces of byte-step records any part_rows-row part spans.
uint32_t rice_part_pieces8(const uint32_t* row_ptr8, uint32_t rows, uint32_t part_rows);
hipError_t launch_rice_apply(const ResView* res_dev, uint32_t n, uint32_t rows, uint32_t cols, uint32_t pieces,
                             const float* x, size_t x_stride, float* y, size_t y_stride, hipStream_t s);
// Device packer (pack_binary_rice_q1): fills the canonical device buffers
// and the host scalars; returns hipErrorInvalidValue if rice_cap is short
// (*rice_bytes then holds the size needed).
struct RicePackResult {
    uint32_t first, k;
    size_t count, rice_bytes;
    uint16_t scale;
    uint32_t bad;  // non-finite input
};
hipError_t pack_binary_rice_device(const float* w, uint32_t rows, uint32_t cols, double ratio, uint16_t* bin_scales,
                                   uint8_t* bin_signs, uint8_t* res_signs, uint8_t* rice, size_t rice_cap,
                                   RicePackResult* out, hipStream_t s);

// Terminal head: the final RMSNorm(1+w) (one block) and the greedy pick.
// key: the caller's 16-byte device slot the pick reduces into (reset by the
// norm, left zeroed by the pick).
hipError_t launch_head_norm(const float* h, const float* w, uint32_t n, float eps, float* xn, int32_t* token,
                            uint64_t* key, uint32_t* status, hipStream_t s);
hipError_t launch_head_argmax(const float* logits, uint32_t n_valid, uint64_t* key, int32_t* token, uint32_t* status,
                              hipStream_t s);
// HGRAVS01 pairs y_i = L_i (R_i x_i) (3-bit factors, right rows = left cols)
// in one launch, one workgroup per pair; mid (may be null) receives R_i x_i.
// lowrank_fusable: the shapes this kernel takes (right cols <= 8192, rank <=
// 2048, LDS within the cap); launch_lowrank returns hipErrorInvalidValue
// otherwise.
bool lowrank_fusable(const OrganView& l, const OrganView& r);
hipError_t launch_lowrank(const OrganView* lefts, const OrganView* rights, uint32_t n, const OrganView& l,
                          const OrganView& r, const float* x, size_t x_stride, float* mid, size_t mid_stride, float* y,
                          size_t y_stride, uint32_t* status, hipStream_t s);
// The fused form for a q8 lm_head of at most 8192 columns: the GEMV forms the
// norm itself and reduces the greedy key (key: 16 zeroed bytes, left zeroed),
// then one pick; h, norm_w and xn 16-byte aligned.
bool head_gemv_fusable(const OrganView& sh);
hipError_t launch_head_fused(const OrganView* organ_dev, const OrganView& sh, const float* h, const float* norm_w,
                             float eps, float* xn, float* logits, uint32_t n_valid, uint64_t* key, int32_t* token,
                             uint32_t* status, hipStream_t s);

// Device bytes of the tiled layout (sections 256-B aligned); mixed needs n_bin/n_q2.
size_t tiled_bytes(int kind, int group, uint32_t rows, uint32_t cols, uint32_t n_bin, uint32_t n_q2,
                   size_t* packed_bytes);
OrganView tiled_place(int kind, int group, uint32_t rows, uint32_t cols, uint32_t n_bin, uint32_t n_q2,
                      uint8_t* base);

}  // namespace hk

// One packed matrix in library-owned device memory (the opaque hk_organ of
// the C ABI).
struct hk_organ {
    hk::OrganView view{};
    int32_t kind = 0;          // the canonical kind it was uploaded as (view.kind is the engine's)
    hk::ResView res{};         // HGRAVR02 residual (res_dev non-null when present)
    void* res_mem = nullptr;
    const hk::ResView* res_dev = nullptr;
    uint32_t res_pieces = 0;   // rice_part_pieces of the residual (RICE_APPLY_ROWS-row parts)
    uint32_t res_pieces_256 = 0;  // the same for 256-row parts
    uint32_t res8_pieces = 0, res8_pieces_256 = 0;  // rice_part_pieces8 of the byte steps, 512- and 256-row parts
    void* view_dev = nullptr;  // device copy of `view` for single-organ launches
    void* mem = nullptr;
    size_t alloc_bytes = 0;
    size_t packed_bytes = 0;
};
