/*
 * hawking_hip.h -- C ABI of the MI355X (gfx950) quantized-decode library.
 *
 * Drop-in boundary for hawking-core's packed-organ / MoE-step compute seam.
 * Citations are path:line inside the reference (joshuahickscorp/hawking),
 * relative to crates/hawking-core/src/.
 *
 * Conventions
 *   - Every entry point returns an int status (HK_OK or an HK_E_* code) and
 *     records a message retrievable with hk_last_error().  Nothing falls back
 *     to the CPU: a missing or failing GPU path is an error, never a silent
 *     substitute (mirrors the fail-closed fallback counters,
 *     model/qwen80_mixed_hybrid_decode.rs:4694-4699,4728-4733).
 *   - Compute entry points take DEVICE pointers, enqueue on the given HIP
 *     stream (hk_stream = hipStream_t; NULL = the null stream), allocate
 *     nothing and never synchronise, like CommandRecorder ops that record
 *     and do not commit (backend/mod.rs:36-41, 227-263).  Geometry is
 *     validated on the host before any launch (the reference kernels
 *     silently no-op on bad geometry, so its hosts validate first).
 *   - Uploads, packers, model/set creation and the helpers marked
 *     "synchronous" allocate and synchronise their stream before they return.
 *   - An hk_ctx is bound to one device and is not thread-safe: one per
 *     host thread.
 */
#ifndef HAWKING_HIP_H
#define HAWKING_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The variants of hawking_core::Error (error.rs:3-27) map as
 * Model -> INVALID_ARG / GEOMETRY / NONFINITE / ROUTE, Metal -> HIP,
 * Unimplemented -> UNSUPPORTED. */
#define HK_OK 0
#define HK_E_INVALID_ARG 1
#define HK_E_GEOMETRY 2
#define HK_E_NONFINITE 3
#define HK_E_HIP 4
#define HK_E_UNSUPPORTED 5
#define HK_E_ROUTE 6
#define HK_E_NOMEM 7

/* Organ kinds: the WeightKind variants the reference's GemvSpec lacks for
 * these formats (backend/mod.rs:120-137, 145-171). */
#define HK_Q4 0    /* uniform Q4, group 32/64/128, f16 scale per group */
#define HK_BIN 1   /* binary sign plane, group 128, f16 mean|w| per group */
#define HK_MIXED 2 /* per-128-group binary | Q2 (two f16 scales per 64) */
#define HK_F32 3   /* dense row-major f32 (router, shared-expert gate) */
#define HK_Q8 4    /* uniform 8-bit, group 64, f16 scale per group (HGRAVU01) */
#define HK_BIN_RICE 6 /* binary group-128 base + Rice-coded 1-bit residual (HGRAVR02);
                         uploaded with hk_organ_upload_rice */
#define HK_U3 5    /* uniform 3-bit, flat groups of 64 (HGRAVS01 low-rank factors);
                      runs on the Q4 engine (nibble = code + 5) */

typedef struct hk_ctx hk_ctx;
typedef struct hk_organ hk_organ;
typedef struct hk_moe_model hk_moe_model;
typedef void* hk_stream;

/* ------------------------------------------------------------------ context */

/* Replaces MetalContext construction (metal/mod.rs:1044). */
int hk_ctx_create(int device, hk_ctx** out);
void hk_ctx_destroy(hk_ctx* ctx);
/* Copies the last error message (NUL-terminated, truncated to len). */
int hk_last_error(const hk_ctx* ctx, char* buf, size_t len);
const char* hk_version(void);
int hk_device_info(hk_ctx* ctx, char* name, size_t len, int* cu_count, size_t* hbm_bytes);

/* ------------------------------------------------ device memory and streams
 * Plumbing for callers without their own allocator; replaces PinnedBuffer /
 * new_buffer_with_bytes_checked (metal/mod.rs:2709-2787).  Copies are
 * stream-ordered; pass the stream and synchronise it before reading. */
int hk_malloc(hk_ctx* ctx, size_t bytes, void** out);
int hk_free(hk_ctx* ctx, void* ptr);
int hk_memcpy_htod(hk_ctx* ctx, void* dst, const void* src, size_t bytes, hk_stream stream);
int hk_memcpy_dtoh(hk_ctx* ctx, void* dst, const void* src, size_t bytes, hk_stream stream);
int hk_memcpy_dtod(hk_ctx* ctx, void* dst, const void* src, size_t bytes, hk_stream stream);
int hk_memset(hk_ctx* ctx, void* dst, int value, size_t bytes, hk_stream stream);
int hk_stream_create(hk_ctx* ctx, hk_stream* out);
int hk_stream_destroy(hk_ctx* ctx, hk_stream stream);
/* The only synchronising calls; TokenCommandBuffer::commit_and_wait (metal/mod.rs:5221). */
int hk_stream_synchronize(hk_ctx* ctx, hk_stream stream);
int hk_device_synchronize(hk_ctx* ctx);
int hk_event_create(hk_ctx* ctx, void** out);
int hk_event_destroy(hk_ctx* ctx, void* event);
int hk_event_record(hk_ctx* ctx, void* event, hk_stream stream);
int hk_event_elapsed_ms(hk_ctx* ctx, void* start, void* stop, float* ms);
/* Synchronises `stream`, returns and clears the device error bits that
 * kernels set when they meet invalid data (1 = non-finite input, 2 = invalid
 * route, 4 = a persistent decode launch gave up waiting for a hand-off).  The GPU-side counterpart of the reference's per-op Result
 * checks, which cannot be returned from stream-ordered launches. */
int hk_check_device_status(hk_ctx* ctx, hk_stream stream, uint32_t* bits);

/* Achievable-bandwidth control, run beside the packed GEMVs to measure what
 * HBM delivers with the same timing (the reference's q80_geo_stream_control,
 * shaders/q80_matvec_geometry_gen.metal:80-107, which its matvec geometry
 * sweep runs beside the organs): reads the nbytes of device memory at data
 * (16-byte aligned, nbytes a multiple of 16) once with 16-byte loads, each
 * of `workgroups` workgroups one contiguous slice, and writes the float sum
 * of each slice's words to out[workgroups] (device).  Stream-ordered. */
int hk_stream_control(hk_ctx* ctx, const void* data, size_t nbytes, float* out, uint32_t workgroups,
                      hk_stream stream);

/* ------------------------------------------------------------------ organs */

/* One packed matrix in the reference's canonical byte layout (HOST memory).
 *  HK_Q4:    scales f16[rows*cols/group] || codes u8[rows*cols/2]
 *            (HQ30UQ4 body, model/qwen_complete_binary/qwen80_uniform_q4.rs:190-278)
 *  HK_BIN:   scales f16[rows*cols/128] || signs u8[rows*cols/8]
 *            (HGRAVB01 body, model/qwen_complete_binary/q80_mixed_decode.rs:185-230)
 *  HK_MIXED: tags u8[ceil(groups/8)], bin_scales f16[n_bin], bin_signs u8[16*n_bin],
 *            q2_scales f16[2*n_q2], q2_codes u8[32*n_q2] (build-defined stream)
 *  HK_F32:   dense f32[rows*cols]
 *  HK_Q8:    scales f16[rows*cols/64] || codes u8[rows*cols], code = q + 127
 *            (HGRAVU01 body, pack_uniform_factor at 8 bits,
 *            model/qwen_complete_binary/q80_mixed_decode.rs:529-577,786-826)
 *  HK_U3:    scales f16[groups] || codes: groups*64 3-bit codes LSB-first,
 *            groups = ceil(rows*cols/64) over the FLAT elements (a group may
 *            span rows; the last is zero-padded), code = q + 3 (HGRAVS01
 *            factor body, pack_uniform_factor at 3 bits); needs cols % 32 == 0.
 * Requires cols % group == 0 (row-aligned groups). */
typedef struct hk_organ_src {
    int32_t kind;
    int32_t group;
    uint32_t rows;
    uint32_t cols;
    const uint16_t* scales;
    const uint8_t* codes;
    const uint8_t* tags;
    const uint16_t* q2_scales;
    const uint8_t* q2_codes;
    uint32_t n_bin;
    uint32_t n_q2;
    const float* dense;
} hk_organ_src;

/* Upload + load-time repack of one organ into library-owned device memory.
 * Replaces Qwen80Q4PackedTensor / MixedPackedTensor::from_codec_payload binds
 * (model/qwen80_uniform_q4_hybrid_decode.rs:957; q80_mixed_decode.rs:1336)
 * and the no-copy bind of payload windows.  Validates geometry and finiteness
 * of every scale.  Synchronous with respect to `stream`'s prior work. */
int hk_organ_upload(hk_ctx* ctx, const hk_organ_src* src, hk_stream stream, hk_organ** out);
int hk_organ_free(hk_ctx* ctx, hk_organ* organ);

/* HGRAVR02 rice_q1_rms body (RiceQ1Packed, q80_mixed_decode.rs:60-69): the
 * binary group-128 base, the outliers' flat indices as `first_index` then
 * Rice-coded gaps (parameter rice_k, LSB-first), one sign bit per outlier
 * (1 = +scale) and one f16 scale.  Pointers may be host or device memory. */
typedef struct hk_rice_q1 {
    uint32_t rows;
    uint32_t cols;                /* multiple of 128, below 32768 */
    const uint16_t* bin_scales;   /* rows*cols/128 */
    const uint8_t* bin_signs;     /* rows*cols/8 */
    uint32_t first_index;
    uint32_t rice_k;
    const uint8_t* rice;          /* rice_bytes (NULL when outlier_count == 1) */
    size_t rice_bytes;
    size_t outlier_count;         /* >= 1 */
    uint16_t residual_scale_f16;
    const uint8_t* residual_signs; /* (outlier_count + 7) / 8 */
} hk_rice_q1;

/* Upload of an HGRAVR02 organ: the base is repacked like a binary organ; the
 * Rice stream is expanded once, on the host at bind time, into a CSR over rows
 * (2 bytes per outlier, rows padded to multiples of four records)
 * (expand_rice_indices + rice_q1_row_ptr, q80_mixed_decode.rs:462-507, and
 * the bind of parse_rice_q1_container, 868-946).  Errors: HK_E_GEOMETRY for
 * a stream that overruns its bytes, a quotient or index above u32, or an index
 * past rows*cols; HK_E_NONFINITE for a non-finite scale.  hk_gemv /
 * hk_gemv_set on the organ compute base + residual
 * (binary_rice_q1_matvec_f32, q80_mixed_decode.rs:509-527). */
int hk_organ_upload_rice(hk_ctx* ctx, const hk_rice_q1* src, hk_stream stream, hk_organ** out);

/* y += (residual of an HGRAVR02 organ) x, adding each row's outliers in index
 * order: the residual half of binary_rice_q1_matvec_f32 and of
 * q80_sparse_q1_apply_csr (shaders/q80_mixed_decode.metal:155-181). */
int hk_rice_apply(hk_ctx* ctx, const hk_organ* organ, const float* x, float* y, hk_stream stream);
int hk_organ_info(const hk_organ* organ, int32_t* kind, int32_t* group, uint32_t* rows,
                  uint32_t* cols, size_t* packed_bytes);

/* y[rows] = W x[cols], f32 in and out (device pointers).
 * Replaces BackendGemv::gemv (backend/mod.rs:270-291) for the packed kinds and
 * the Q4/binary matvec kernels (shaders/qwen_uniform_q4.metal:183-272,
 * shaders/q80_mixed_decode.metal:701-741).  Numerics: within 2e-5 relative L2
 * of Qwen80Q4PackedTensor::matvec / binary_group_matvec_f32. */
int hk_gemv(hk_ctx* ctx, const hk_organ* organ, const float* x, float* y, hk_stream stream);

/* SYNCHRONOUS helper: n organs of one kind and shape in ONE launch,
 * y_i = W_i x_i with x_i = x + i*x_stride, y_i = y + i*y_stride (element
 * strides).  The batched form of matvec_batch (gravity_glm.rs:515-548).  It
 * builds a transient organ set (device allocation and a blocking copy),
 * launches, synchronises `stream` and frees the set: stream-ordered callers
 * create the set once (hk_organ_set_create) and call hk_gemv_set. */
int hk_gemv_batch(hk_ctx* ctx, const hk_organ* const* organs, uint32_t n, const float* x,
                  size_t x_stride, float* y, size_t y_stride, hk_stream stream);

/* A fixed set of organs of one kind and shape whose device descriptor table
 * is uploaded once, so hk_gemv_set launches with no host synchronisation
 * (the persistent form of the routed wave / matvec_batch). */
typedef struct hk_organ_set hk_organ_set;
int hk_organ_set_create(hk_ctx* ctx, const hk_organ* const* organs, uint32_t n, hk_organ_set** out);
int hk_organ_set_free(hk_ctx* ctx, hk_organ_set* set);
/* y_i = W_i x_i for every organ of the set in ONE launch (strides as hk_gemv_batch). */
int hk_gemv_set(hk_ctx* ctx, const hk_organ_set* set, const float* x, size_t x_stride, float* y,
                size_t y_stride, hk_stream stream);

/* HGRAVS01 low-rank organ: mid[rank] = right x, then y[rows] = left mid (mid
 * is a caller buffer of rank floats, 16-byte aligned, and receives R x).  The
 * factors are HK_U3 organs (left rows x rank, right rank x cols); one launch
 * when cols <= 8192 and rank <= 2048, else two ordered on `stream`.
 * Replaces hgravs01_two_stage_matvec_f32 (q80_mixed_decode.rs:614-629). */
int hk_gemv_lowrank(hk_ctx* ctx, const hk_organ* left, const hk_organ* right, const float* x,
                    float* mid, float* y, hk_stream stream);
/* y_i = L_i (R_i x_i) for the n HGRAVS01 pairs of two organ sets (left set of
 * HK_U3 rows x rank, right set of HK_U3 rank x cols, the same n), streamed in
 * ONE launch (one workgroup per pair, mid kept on chip) for the shapes
 * hk_gemv_lowrank fuses, else two set launches ordered on `stream` through
 * mid.  mid (device, mid_i = mid + i*mid_stride, 16-byte aligned) may be
 * NULL when the pair is fused; when given it receives R_i x_i; the two-launch
 * shapes (right cols > 8192 or rank > 2048) require it (HK_E_INVALID_ARG).
 * Strides as hk_gemv_batch.  The set form of hgravs01_two_stage_matvec_f32
 * (q80_mixed_decode.rs:614-629) over a routed wave's down projections. */
int hk_gemv_lowrank_set(hk_ctx* ctx, const hk_organ_set* left, const hk_organ_set* right, const float* x,
                        size_t x_stride, float* mid, size_t mid_stride, float* y, size_t y_stride,
                        hk_stream stream);

/* Bit-exact decode probe: out[nrows*cols] = decoded weights of rows
 * [row0, row0+nrows).  Replaces qwen_uniform_q4_decode_vector
 * (shaders/qwen_uniform_q4.metal:627) and gather_row
 * (model/qwen80_uniform_q4_hybrid_decode.rs:900-911).  An HGRAVR02 organ
 * decodes to its base plus +-scale at each outlier. */
int hk_decode_rows(hk_ctx* ctx, const hk_organ* organ, uint32_t row0, uint32_t nrows,
                   float* out, hk_stream stream);

/* ------------------------------------------- device packers and generator
 * Bit-exact with the reference packers on the same f32 input (device
 * pointers in and out). */
/* pack_uniform_q4_group64 (qwen80_uniform_q4.rs:190-278), group 32/64/128. */
int hk_pack_q4(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, int32_t group,
               uint16_t* scales, uint8_t* codes, hk_stream stream);
/* pack_binary_group (q80_mixed_decode.rs:185-230), group 128. */
int hk_pack_bin(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, uint16_t* scales,
                uint8_t* signs, hk_stream stream);
/* pack_uniform_factor at 8 bits, group 64 (q80_mixed_decode.rs:529-577);
 * cols % 64 == 0.  An f16 scale that overflows is reported as HK_E_NONFINITE. */
int hk_pack_q8(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, uint16_t* scales, uint8_t* codes,
               hk_stream stream);
/* pack_uniform_factor at 3 bits, group 64, over `count` flat values (the
 * HGRAVS01 factor codec, q80_mixed_decode.rs:529-577): scales f16[ceil(count/64)],
 * codes 24 bytes per group (16-byte aligned). */
int hk_pack_u3(hk_ctx* ctx, const float* w, size_t count, uint16_t* scales, uint8_t* codes,
               hk_stream stream);
/* pack_binary_rice_q1 (q80_mixed_decode.rs:383-460) on the device: w
 * (device, rows x cols, cols % 128 == 0) -> bin_scales [rows*cols/128],
 * bin_signs [rows*cols/8], residual_signs [(count+7)/8] and the Rice stream in
 * rice (16-byte aligned, rice_cap bytes; the writer needs the stream rounded
 * up to whole 4-byte words).  *out receives the scalars and these pointers.
 * outlier_ratio in (0, 0.1]; count = clamp(ceil(n * ratio), 1, n).  A short
 * rice_cap fails with HK_E_INVALID_ARG and out->rice_bytes = the size needed. */
int hk_pack_binary_rice(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, double outlier_ratio,
                        uint16_t* bin_scales, uint8_t* bin_signs, uint8_t* residual_signs, uint8_t* rice,
                        size_t rice_cap, hk_rice_q1* out, hk_stream stream);
/* Q2 base stage of _additive_residual_codec
 * (lab/operators/ascension_dual_gravity_worker.py:898-911), group 64. */
int hk_pack_q2(hk_ctx* ctx, const float* w, size_t count, uint16_t* scales, uint8_t* codes,
               hk_stream stream);
/* The per-group mixed packer (HK_MIXED, build-defined stream; no reference
 * counterpart packs per group -- the reference mixes codecs per tensor,
 * q80_mixed_decode.rs:1073-1417): w (device, rows x cols f32, cols % 128 ==
 * 0) in flat groups of 128; group g is packed by pack_binary_group
 * (q80_mixed_decode.rs:185-230) when is_binary[g] != 0 (device u8 per
 * group), else by the Q2 base stage on each half of 64
 * (ascension_dual_gravity_worker.py:898-911), into the canonical stream of
 * hk_organ_src: tags [(groups + 7) / 8] (1 = binary, LSB-first), bin_scales
 * [n_bin] and bin_signs [16 n_bin] (16-byte aligned), q2_scales [2 n_q2] and
 * q2_codes [32 n_q2] (16-byte aligned), sections in group order.  *n_bin_out
 * receives n_bin; a selector with more binary (Q2) groups than bin_cap
 * (q2_cap) fails with HK_E_INVALID_ARG before anything past the tags is
 * written.  Bit-exact with the oracle's mixed pack; synchronous. */
int hk_pack_mixed(hk_ctx* ctx, const float* w, uint32_t rows, uint32_t cols, const uint8_t* is_binary,
                  uint8_t* tags, uint16_t* bin_scales, uint8_t* bin_signs, uint32_t bin_cap, uint16_t* q2_scales,
                  uint8_t* q2_codes, uint32_t q2_cap, uint32_t* n_bin_out, hk_stream stream);
/* Synthetic N(0, sigma): counter-based SplitMix64 words -> Irwin-Hall(12),
 * integer-exact so host and device draws agree bit for bit.  No reference
 * counterpart (the reference's synthetic inputs are deterministic_matrix /
 * deterministic_input, q80_mixed_decode.rs:631-647). */
uint64_t hk_stream_key(uint64_t seed, uint64_t stream_id);
int hk_synth_normal(hk_ctx* ctx, uint64_t key, uint64_t first, size_t count, float sigma,
                    float* out, hk_stream stream);

/* One organ generated and packed on the device: weights synth_normal(key, e, sigma)
 * in row-major order, mixed coins from coin_key (as the MoE synthetic fill). */
int hk_organ_synthetic(hk_ctx* ctx, int32_t kind, int32_t group, uint32_t rows, uint32_t cols,
                       uint64_t key, uint64_t coin_key, float sigma, hk_stream stream,
                       hk_organ** out);

/* ------------------------------------------------------------ containers */

/* Codec ids of the mixed catalog (qwen80_mixed_catalog.rs:30-33). */
#define HK_CODEC_BINARY 0   /* HGRAVB01 binary_sign_scale, group 128 */
#define HK_CODEC_RESIDUAL 1 /* HGRAVR02 binary + Rice-coded 1-bit residual */
#define HK_CODEC_HGRAVS01 2 /* low-rank, two uniform factors (3-bit G64 on the device) */
#define HK_CODEC_UNIFORM8 3 /* HGRAVU01 uniform q8 G64 */

/* One HGRAV* container payload (host memory: 8-byte magic, u32 LE JSON header
 * length, JSON header, body) parsed and validated as
 * MixedPackedTensor::from_codec_payload does (q80_mixed_decode.rs:135-147,
 * 823-1070,1336-1347) and bound: HGRAVB01 -> HK_BIN, HGRAVU01 -> HK_Q8,
 * HGRAVR02 -> an HGRAVR02 organ, HGRAVS01 -> *out = the left factor and
 * *right = the right one (HK_U3; use hk_gemv_lowrank).  right may be NULL
 * except for HGRAVS01.  Errors: HK_E_INVALID_ARG (magic, JSON, schema,
 * missing fields), HK_E_GEOMETRY (ledgers, shapes), HK_E_UNSUPPORTED (valid
 * for the reference but not a device kind here: HGRAVS01 factors other than
 * 3-bit G64, binary groups other than 128). */
int hk_organ_from_container(hk_ctx* ctx, int32_t codec, const uint8_t* payload, size_t len, hk_stream stream,
                            hk_organ** out, hk_organ** right);

/* An HQ30UQ4 (uniform Q4, group 64/128) or HQ30G1B1 (binary) payload with its
 * 32-byte header (parse_uniform_q4_header, qwen_complete_binary/uniform_q4.rs:57-150;
 * parse_complete_binary_header, qwen_complete_binary/mod.rs:137-233) bound as
 * an HK_Q4 / HK_BIN organ; shape [rows, cols] or [len] (= len x 1). */
int hk_organ_from_hq30(hk_ctx* ctx, const uint8_t* payload, size_t len, hk_stream stream, hk_organ** out);

/* GGUF Q4_0 (dequant_q4_0, quant.rs:473-498): rows*cols/32 AoS blocks of 18
 * bytes {f16 d (LE); u8 qs[16]} (HOST memory, row-major, blocks along each
 * row; cols % 32 == 0), element j of a block in the low nibble of qs[j] for
 * j < 16 and in the high nibble of qs[j - 16] for j >= 16, value
 * (nibble - 8) * d.  Bound as an HK_Q4 group-32 organ (the same d and
 * nibbles, reordered into the canonical even/odd pairs), so it decodes bit
 * for bit to dequant_q4_0.  Errors: HK_E_GEOMETRY (shape, cols % 32, len !=
 * rows*cols/32*18), HK_E_NONFINITE (a d that is not a finite f16). */
int hk_organ_from_q4_0(hk_ctx* ctx, const uint8_t* blocks, size_t len, uint32_t rows, uint32_t cols,
                       hk_stream stream, hk_organ** out);

/* The HQ80M15 mixed catalog (Qwen80MixedStreamingCatalog,
 * qwen80_mixed_catalog.rs:176-555): the manifest JSON (schema, seal, bpw
 * ledger, catalog path + SHA-256, checked), the catalog's segment table and
 * 128-byte tensor records; payloads are windows of memory-mapped
 * <manifest dir>/segments/<file>. */
typedef struct hk_catalog hk_catalog;
typedef struct hk_catalog_record {
    const char* name;       /* valid while the catalog is open */
    uint32_t codec, organ, ndim;
    uint32_t shape[4];
    uint64_t elements;
    uint16_t segment_id, achieved_rank;
    uint64_t offset, nbytes;
    uint8_t sha256[32];
    uint32_t flags, n_fit_rows;
    float codec_bpw;
} hk_catalog_record;
int hk_catalog_open(hk_ctx* ctx, const char* manifest_path, hk_catalog** out);
int hk_catalog_close(hk_catalog* catalog);
int hk_catalog_info(const hk_catalog* catalog, uint32_t* n_tensors, uint32_t* n_segments,
                    double* complete_physical_bpw, uint64_t* tensor_payload_bytes);
int hk_catalog_record_at(const hk_catalog* catalog, uint32_t index, hk_catalog_record* out);
int hk_catalog_find(hk_ctx* ctx, const hk_catalog* catalog, const char* name, hk_catalog_record* out);
/* The tensor's payload window (valid while the catalog is open); with
 * verify_sha256 its SHA-256 is checked against the record on first use. */
int hk_catalog_payload(hk_ctx* ctx, hk_catalog* catalog, const char* name, int verify_sha256, const uint8_t** data,
                       size_t* len);
/* load_packed: the payload through hk_organ_from_container by its codec. */
int hk_catalog_load(hk_ctx* ctx, hk_catalog* catalog, const char* name, int verify_sha256, hk_stream stream,
                    hk_organ** out, hk_organ** right);

/* ------------------------------------------------------------ terminal head */

/* terminal_greedy on the device (model/qwen80_mixed_hybrid_decode.rs:3754-3790):
 * xn = RMSNorm(1+w)(hidden) (source_qwen80_residual_rms_norm,
 * model/qwen80_complete_runtime.rs:6778-6797), logits = lm_head xn (any organ
 * kind; the reference's mixed pack stores it as HGRAVU01 q8 G64), and
 * token = the lowest index of the largest non-NaN logit among the first
 * n_valid (the rows past the tokenizer's vocabulary are never chosen).  All
 * pointers are device memory: hidden and norm_w [lm_head cols], xn [cols] and
 * logits [lm_head rows] are caller workspaces (16-byte aligned), pick a
 * 16-byte caller workspace (8-byte aligned) the greedy key reduces into,
 * which must hold zeros before its first use and which every call leaves
 * zeroed, token one int32.  A non-finite xn or a best logit that is not
 * finite writes token -1 and latches HK_E_NONFINITE in the device status
 * (hk_check_device_status), where the reference returns an error.
 * Stream-ordered, no host round trip; the lm_head organ is only read, so
 * calls with separate workspaces may share it across streams. */
int hk_terminal_greedy(hk_ctx* ctx, const float* hidden, const float* norm_w, float eps, const hk_organ* lm_head,
                       uint32_t n_valid, float* xn, float* logits, uint64_t* pick, int32_t* token,
                       hk_stream stream);

/* NO reference counterpart: hk_terminal_greedy for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc): the same result with the xn, logits and pick workspaces in a
 * library-owned static device array of 1 MiB + 32 KiB + 256 B per device,
 * held until the process ends.  Limits: lm_head rows <= HK_NOALLOC_HEAD_MAX_ROWS,
 * cols <= HK_NOALLOC_HEAD_MAX_COLS (HK_E_UNSUPPORTED beyond).  Allocates
 * nothing.  Every call on a device shares that device's array, which keeps
 * the last call's xn and logits: calls that overlap on one device race (use
 * one stream, or synchronised streams). */
#define HK_NOALLOC_HEAD_MAX_ROWS 262144
#define HK_NOALLOC_HEAD_MAX_COLS 8192
int hk_terminal_greedy_noalloc(hk_ctx* ctx, const float* hidden, const float* norm_w, float eps,
                               const hk_organ* lm_head, uint32_t n_valid, int32_t* token, hk_stream stream);

/* ------------------------------------------------------------------ routers */

/* Per token: softmax over n_experts logits, top_k by strict '>' (lowest index
 * on exact ties; tie_eps > 0 = HAWKING_DS_ROUTE_TIE_EPS window), renormalised
 * by the selected sum.  ids/weights stay on the device.
 * source_qwen80_topk_router (model/qwen80_complete_runtime.rs:5970-6025),
 * moe_topk_gate (shaders/moe.metal:118-305, kernels/mod.rs:12721-12790).
 * renorm = 0 gives topk_softmax_batch (kernels/mod.rs:342-374).
 * Limits: n_experts <= 8192, top_k <= 64 (HK_E_UNSUPPORTED beyond). */
int hk_router_softmax_topk(hk_ctx* ctx, const float* logits, uint32_t n_tokens,
                           uint32_t n_experts, uint32_t top_k, float tie_eps, int renorm,
                           int32_t* ids, float* weights, hk_stream stream);
/* noaux_tc (gravity_glm.rs:447-500): select on sigmoid(logit)+bias inside the
 * top topk_group groups (group score = sum of its best two), weight with the
 * uncorrected sigmoid, optional renorm (+1e-20), times routed_scaling_factor.
 * Limits: n_experts <= 8192, top_k <= 64. */
int hk_router_noaux_tc(hk_ctx* ctx, const float* logits, const float* bias, uint32_t n_tokens,
                       uint32_t n_experts, uint32_t n_group, uint32_t topk_group, uint32_t top_k,
                       int norm_topk_prob, float routed_scaling_factor, int32_t* ids,
                       float* weights, hk_stream stream);

/* ------------------------------------------------------------------ MoE step */

/* Router kinds of an MoE model. */
#define HK_ROUTER_SOFTMAX 0  /* softmax, top-k, renormalise (source_qwen80_topk_router) */
#define HK_ROUTER_NOAUX_TC 1 /* sigmoid + bias, group-limited top-k (gravity_glm.rs:447-500) */

typedef struct hk_moe_config {
    uint32_t n_layers;
    uint32_t hidden;
    uint32_t inter;          /* routed expert intermediate */
    uint32_t shared_inter;   /* 0 = no shared expert */
    uint32_t n_experts;
    uint32_t top_k;
    int32_t expert_kind;     /* HK_Q4 or HK_MIXED */
    int32_t expert_group;    /* Q4 group (32/64/128); 128 for mixed */
    int32_t shared_gate;     /* 1 = sigmoid(wg . xn) gate on the shared expert */
    float eps;               /* RMSNorm epsilon */
    int32_t router;          /* HK_ROUTER_SOFTMAX (decode path) or HK_ROUTER_NOAUX_TC (batched path) */
    uint32_t n_group;        /* noaux_tc: expert groups (n_experts % n_group == 0) */
    uint32_t topk_group;     /* noaux_tc: groups kept */
    int32_t norm_topk_prob;  /* noaux_tc: renormalise the selected scores (+1e-20) */
    float routed_scaling_factor; /* noaux_tc: factor on the routed weights */
    float route_tie_eps;     /* softmax router: the HAWKING_DS_ROUTE_TIE_EPS window (route_tie_epsilon,
                                moe.rs:8-14): a later probability replaces the best only when it is above
                                it by more than this; 0 = strict '>' with the lowest index on exact ties */
    int32_t stack_launch;    /* hk_moe_decode_stack: HK_STACK_PER_LAYER or HK_STACK_PERSISTENT */
} hk_moe_config;

/* How hk_moe_decode_stack runs a token (hk_moe_config.stack_launch). */
#define HK_STACK_PER_LAYER 0  /* three stream-ordered launches per layer */
#define HK_STACK_PERSISTENT 1 /* one persistent cooperative launch for every layer (the reference's one command
                                 buffer per token, qwen80_mixed_hybrid_decode.rs:1962-2078) when its grid can
                                 be resident at once, else the per-layer launches; the same bits either way */

/* Host-side canonical weights of one layer (HOST pointers).
 * experts: n_experts*3 organ sources (gate, up, down per expert). */
typedef struct hk_moe_layer_src {
    const float* norm_w;         /* [hidden], applied as (1 + w) (decode path) */
    const float* router_w;       /* [n_experts x hidden] f32 */
    const float* shared_gate_w;  /* [hidden] or NULL */
    const hk_organ_src* experts; /* [n_experts*3] */
    const hk_organ_src* shared;  /* [3] or NULL */
    const float* router_bias;    /* [n_experts] e_score_correction_bias (noaux_tc), else NULL */
} hk_moe_layer_src;

/* Expert table + per-layer dense weights in device memory: each expert's
 * gate|up|down laid out contiguously (Qwen80DeviceExpertTriplet,
 * model/qwen80_device_expert_table.rs:116-156).
 * Limits (HK_E_UNSUPPORTED beyond): top_k + (1 if shared_inter) <= 16 (one
 * wave per slot in the down kernel), n_experts <= 4096 (<= 512 for
 * HK_ROUTER_NOAUX_TC), hidden % 128 == 0 and hidden <= 8192, and the x
 * images of hidden / intermediate within 64 KiB of LDS. */
int hk_moe_model_create(hk_ctx* ctx, const hk_moe_config* cfg, hk_moe_model** out);
int hk_moe_model_free(hk_ctx* ctx, hk_moe_model* model);
int hk_moe_model_set_layer(hk_ctx* ctx, hk_moe_model* model, uint32_t layer,
                           const hk_moe_layer_src* src, hk_stream stream);
/* Generate every layer on the device with the synthetic generator (layer l,
 * expert e, projection p draw stream hk_moe_stream_id(l, e, p)). */
int hk_moe_model_fill_synthetic(hk_ctx* ctx, hk_moe_model* model, uint64_t seed,
                                hk_stream stream);
/* stream id = ((layer+1) << 40) | (expert << 8) | proj; proj 0/1/2 = gate/up/down,
 * 16 = norm weight, 17 = router, 18 = shared-expert gate, 19 = router bias (N(0, 0.01)),
 * 32+p = mixed coins of proj p; expert n_experts = the shared expert. */
uint64_t hk_moe_stream_id(uint32_t layer, uint32_t expert, uint32_t proj);
/* Device bytes held by the model; dense (norm + router + gate) bytes read per layer. */
int hk_moe_model_bytes(const hk_moe_model* model, size_t* device_bytes, size_t* dense_bytes_per_layer);
/* Packed (algorithmic) bytes of one expert's gate+up+down; expert n_experts = shared. */
int hk_moe_expert_bytes(const hk_moe_model* model, uint32_t layer, uint32_t expert, size_t* bytes);

/* One moe_suffix layer at batch 1 on device data, no host round trip
 * (router == HK_ROUTER_SOFTMAX):
 * xn = RMSNorm(1+w)(h); logits = Wr xn; route = softmax top-k renorm;
 * out = h + sum_r w_r mlp_r(xn) (route order) + g * mlp_shared(xn).
 * (model/qwen80_uniform_q4_hybrid_decode.rs:2615-2757,
 *  run_qwen80_routed_expert_table model/qwen80_device_expert_table.rs:1204-1247,
 *  routed_wave_fused model/qwen80_mixed_hybrid_decode.rs:1962-2078.)
 * ids/weights (device, top_k each) may be NULL. */
int hk_moe_decode_layer(hk_ctx* ctx, hk_moe_model* model, uint32_t layer, const float* h_in,
                        float* h_out, int32_t* ids, float* weights, hk_stream stream);
/* All layers for one token: h_{l+1} = moe_layer_l(h_l) (forward_token's MoE
 * suffixes, model/qwen80_mixed_hybrid_decode.rs:4682-4736, without the
 * attention mixers).  ids/weights may be NULL or [n_layers*top_k].  Runs as
 * three launches per layer (stack_launch = HK_STACK_PER_LAYER), or, with
 * HK_STACK_PERSISTENT, as one persistent cooperative launch (the reference's
 * one command buffer per token) when the model's grid fits the device at once
 * (hidden <= 2048, n_experts <= 512, intermediate <= 2048, top_k + shared <=
 * 12); both give the same bits.  A hand-off the persistent launch waited for
 * too long sets device status bit 4: h_out, ids and weights of that call are
 * then undefined (the next call, with a new tag, is unaffected). */
int hk_moe_decode_stack(hk_ctx* ctx, hk_moe_model* model, const float* h_in, float* h_out,
                        int32_t* ids, float* weights, hk_stream stream);
/* *persistent = 1 when hk_moe_decode_stack on this model runs as one
 * persistent launch (selected and admitted), 0 when it uses per-layer launches.  Diagnostic with no
 * counterpart in the reference (its token is one command buffer). */
int hk_moe_decode_stack_persistent(hk_ctx* ctx, hk_moe_model* model, int* persistent);
/* Changes the model's hk_moe_config.stack_launch after creation (HK_STACK_PER_LAYER or
 * HK_STACK_PERSISTENT); no reference counterpart.  Not to be called while a token of the
 * model is in flight on another stream. */
int hk_moe_model_set_stack_launch(hk_ctx* ctx, hk_moe_model* model, int32_t stack_launch);
/* The persistent launch's bound on each hand-off wait: a wait that has polled
 * `polls` times without its producer's words gives up, sets device status
 * bit 4 (value 4, hk_check_device_status) and makes every other wait of that launch return,
 * so the launch always ends; h_out, ids and weights of that call are then
 * undefined and the next call (a new tag) is unaffected.  Default
 * HK_STALL_POLLS_DEFAULT (tens of milliseconds); 0 gives up at the first
 * wait that finds its words missing.  No reference counterpart (its command
 * buffer has no hand-off waits).  Not to be called while a token of the model
 * is in flight on another stream. */
#define HK_STALL_POLLS_DEFAULT 65536u
int hk_moe_model_set_stall_polls(hk_ctx* ctx, hk_moe_model* model, uint32_t polls);

/* BackendMoe::moe_block (backend/mod.rs:509-521) on one layer of a model:
 * the routed (and optional shared) expert block for CALLER-supplied routes,
 * accumulated into out:
 *   combined = sum_r w_r mlp_{id_r}(x)   (route order, r < n_routes)
 *              + g * mlp_shared(x)        (include_shared and a shared expert;
 *                                          g = sigmoid(shared_gate . x), or 1
 *                                          for a model without the gate)
 *   out = out + combined
 * with mlp(x) = down(silu(gate x) * up x).  x is the block input (no
 * RMSNorm, no router here); route_ids (int32) and route_weights (f32) are
 * device arrays of n_routes entries, 1 <= n_routes <= the model's top_k.
 * With include_shared = 0 and out zeroed this is
 * run_qwen80_routed_expert_table's combined
 * (model/qwen80_device_expert_table.rs:1204-1247, weighted_sum
 * shaders/qwen80_device_expert_table.metal:430-446); moe_suffix is RMSNorm,
 * the router (hk_router_softmax_topk) and this block with out = h.  An id
 * outside [0, n_experts) contributes nothing and latches HK_E_ROUTE's device
 * bit (hk_check_device_status).  x and out are device vectors of hidden
 * floats, 16-byte aligned, and may be the same vector.  Two launches, no
 * host round trip; calls on one model share its workspace and must not
 * overlap. */
int hk_moe_block(hk_ctx* ctx, hk_moe_model* model, uint32_t layer, const int32_t* route_ids,
                 const float* route_weights, uint32_t n_routes, int include_shared, const float* x, float* out,
                 hk_stream stream);

/* The noaux_tc MoE block for a batch of tokens (routed_moe, gravity_glm.rs:550-600,
 * with batched_mlp :515-548): per token t, logits = Wr x_t; route = noaux_tc;
 * y_t = sum over the routed experts in ascending id of w_e mlp_e(x_t), then
 * + mlp_shared(x_t).  x is the block input (no norm, no residual), bf16
 * [n_tokens x hidden] (device); y f32 [n_tokens x hidden] (device); ids/weights
 * [n_tokens x top_k] (device, route order) may be NULL.  Each active expert's
 * weights are streamed once for all of its tokens (grouped expert GEMM).
 * Requires router == HK_ROUTER_NOAUX_TC, expert_kind == HK_Q4, no shared gate,
 * n_tokens <= 64, n_experts <= 512, x and y 16-byte aligned.  The workspace
 * (for 64 tokens) is allocated with the model; calls on one model must not
 * overlap. */
int hk_moe_forward_batch(hk_ctx* ctx, hk_moe_model* model, uint32_t layer, const uint16_t* x_bf16,
                         uint32_t n_tokens, float* y, int32_t* ids, float* weights, hk_stream stream);

/* ------------------------------------------------- mixed-1p5 MoE layer */

/* One MoE layer of the mixed-1p5-v1 artifact built from bound organs (the
 * library keeps pointers to them: free the layer before its organs).
 * Routed expert e: gate[e] HGRAVB01 (HK_BIN, inter x hidden), up[e] HGRAVR02
 * (inter x hidden), down = down_left[e] (hidden x rank) . down_right[e]
 * (rank x inter), the HGRAVS01 factors.  Router (n_experts x hidden),
 * shared_gate (1 x hidden), shared_gate_proj / shared_up (shared_inter x
 * hidden) and shared_down (hidden x shared_inter): any non-residual kind,
 * HGRAVU01 q8 in the artifact.  shared_inter = 0: no shared expert (its
 * organs may be NULL).  norm_w is a HOST pointer [hidden]. */
typedef struct hk_moe15_layer hk_moe15_layer;
typedef struct hk_moe15_layer_src {
    uint32_t hidden, inter, shared_inter, n_experts, top_k;
    float eps;
    float route_tie_eps;   /* as hk_moe_config.route_tie_eps (0 = strict '>') */
    const float* norm_w;
    const hk_organ* router;
    const hk_organ* shared_gate;
    const hk_organ* shared_gate_proj;
    const hk_organ* shared_up;
    const hk_organ* shared_down;
    const hk_organ* const* gate;       /* [n_experts] */
    const hk_organ* const* up;         /* [n_experts] */
    const hk_organ* const* down_left;  /* [n_experts] */
    const hk_organ* const* down_right; /* [n_experts] */
} hk_moe15_layer_src;
/* Limits: top_k <= 16 (and <= n_experts), n_experts <= 512, hidden a
 * multiple of 64 and at most 8192, inter a multiple of 4, each kernel's LDS
 * within 64 KiB (HK_E_UNSUPPORTED / HK_E_GEOMETRY otherwise). */
int hk_moe15_layer_create(hk_ctx* ctx, const hk_moe15_layer_src* src, hk_moe15_layer** out);
int hk_moe15_layer_free(hk_ctx* ctx, hk_moe15_layer* layer);
/* moe_suffix of the mixed decode (model/qwen80_mixed_hybrid_decode.rs:3636-3752
 * with routed_wave :2192-2386) at batch 1 on device data:
 * xn = RMSNorm(1+w)(h); route = softmax top-k renorm of router xn;
 * act_r = silu(gate_r xn) * (up_r xn); y_r = L_r (R_r act_r);
 * out = h + sum_r w_r y_r (route order) + sigmoid(shared_gate xn) * shared(xn).
 * ids/weights (device, top_k each) may be NULL.  Stream-ordered, no sync;
 * layer workspace is reused, so calls on one layer must not overlap. */
int hk_moe15_decode_layer(hk_ctx* ctx, hk_moe15_layer* layer, const float* h, float* out, int32_t* ids,
                          float* weights, hk_stream stream);
/* n_layers layers for one token, h_{l+1} = layer_l(h_l) (forward_token's MoE
 * suffixes, model/qwen80_mixed_hybrid_decode.rs:4682-4736, without the
 * attention mixers); the intermediate states live in the layers' workspace.
 * Layers share hidden and top_k; ids/weights may be NULL or [n_layers*top_k]. */
int hk_moe15_decode_stack(hk_ctx* ctx, hk_moe15_layer* const* layers, uint32_t n_layers, const float* h, float* out,
                          int32_t* ids, float* weights, hk_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* HAWKING_HIP_H */
