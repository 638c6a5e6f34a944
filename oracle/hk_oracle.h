/*
 * hk_oracle.h -- CPU oracle for the quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * CPU path (joshuahickscorp/hawking, crate hawking-core).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker or the timed CPU baseline; the product library
 * (hawking_amd/) never links or calls it.
 *
 * Build flags matter: -O2 -ffp-contract=off, no -ffast-math.  Rust never
 * fuses a*b+c, so every f32 expression below is evaluated op by op with
 * IEEE round-to-nearest-even, in the reference's order.  exp() is glibc
 * expf, which is what Rust's f32::exp calls on Linux.
 *
 * Citations are path:line relative to the reference root.
 */
#ifndef HK_ORACLE_H
#define HK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (same numbering as the product's C ABI). */
#define HKO_OK 0
#define HKO_E_INVALID_ARG 1
#define HKO_E_GEOMETRY 2
#define HKO_E_NONFINITE 3
#define HKO_E_UNSUPPORTED 5
#define HKO_E_ROUTE 6

/* ---- IEEE binary16 (the `half` 2.7.1 crate's from_f32 / to_f32) ---- */
uint16_t hko_f32_to_f16(float value);
float hko_f16_to_f32(uint16_t bits);
/* IEEE roundTiesToEven on f32, restating rint_ties_even
 * (crates/hawking-core/src/model/qwen_complete_binary/qwen80_uniform_q4.rs:170-188). */
float hko_rint_ties_even(float value);

/* ---- reference deterministic generators
 * (crates/hawking-core/src/model/qwen_complete_binary/q80_mixed_decode.rs:631-647) ---- */
void hko_deterministic_matrix(size_t rows, size_t cols, uint32_t seed, float* out);
void hko_deterministic_input(size_t cols, float* out);

/* ---- synthetic N(0, sigma) generator shared with the GPU generator:
 * counter-based SplitMix64 words -> Irwin-Hall(12) normal, integer-exact,
 * so the CPU and the GPU draw bit-identical f32 values. ---- */
uint64_t hko_stream_key(uint64_t seed, uint64_t stream);
float hko_normal(uint64_t key, uint64_t index, float sigma);
void hko_fill_normal(uint64_t key, size_t count, float sigma, float* out);
/* elements [first, first+count) of the stream */
void hko_fill_normal_from(uint64_t key, uint64_t first, size_t count, float sigma, float* out);
/* 1 when the 128-group `group` (flat index) of a mixed tensor is binary. */
int hko_mixed_coin(uint64_t coin_key, uint64_t group);
void hko_fill_coins(uint64_t coin_key, size_t groups, uint8_t* out);

/* ---- Q4 uniform (HQ30UQ4 semantics, SoA: f16 scales[groups] || codes[groups*G/2]).
 * Packer: pack_uniform_q4_group64 (qwen80_uniform_q4.rs:190-278) with G in {32,64,128};
 * decode: decode_uniform_q4_group64 (qwen80_uniform_q4.rs:325-346);
 * matvec: Qwen80Q4PackedTensor::matvec (qwen80_uniform_q4_hybrid_decode.rs:957-1036). ---- */
int hko_q4_pack(const float* w, size_t rows, size_t cols, int group,
                uint16_t* scales, uint8_t* codes);
int hko_q4_decode(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols,
                  int group, float* out);
int hko_q4_matvec(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols,
                  int group, const float* x, float* y);
int hko_q4_matvec_f64(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols,
                      int group, const double* x, double* y);
/* GGUF Q4_0 array-of-structs blocks {f16 d; u8 qs[16]}: dequant_q4_0 (src/quant.rs:473-498). */
int hko_q4_0_dequant(const uint8_t* blocks, size_t elements, float* out);

/* ---- binary sign plane, group 128 (HGRAVB01 body: f16 scales || LSB-first signs).
 * pack_binary_group / binary_group_matvec_f32 (q80_mixed_decode.rs:185-257). ---- */
int hko_bin_pack(const float* w, size_t rows, size_t cols, int group,
                 uint16_t* scales, uint8_t* signs);
int hko_bin_decode(const uint16_t* scales, const uint8_t* signs, size_t rows, size_t cols,
                   int group, float* out);
int hko_bin_matvec(const uint16_t* scales, const uint8_t* signs, size_t rows, size_t cols,
                   int group, const float* x, float* y);
int hko_bin_matvec_f64(const uint16_t* scales, const uint8_t* signs, size_t rows, size_t cols,
                       int group, const double* x, double* y);

/* ---- Q2 stage, group 64: scale=f16(max|w|/1.5), code=clip(rint(w/scale+1.5),0,3),
 * 2-bit LSB-first codes (lab/operators/ascension_dual_gravity_worker.py:849-936,
 * pack_unsigned q80_mixed_decode.rs:170-183). ---- */
int hko_q2_pack(const float* w, size_t count, uint16_t* scales, uint8_t* codes);
int hko_q2_decode(const uint16_t* scales, const uint8_t* codes, size_t count, float* out);

/* ---- uniform factor codec: HGRAVU01 (q8, group 64) and the HGRAVS01 low-rank
 * factors (3-bit, group 64); pack_uniform_factor / uniform_factor_value /
 * uniform_factor_matvec_f32 / hgravs01_two_stage_matvec_f32
 * (q80_mixed_decode.rs:529-629).  scales f16[groups] (flat groups, last one
 * padded with zeros), codes = (groups*group) codes of `bits` bits, LSB-first. ---- */
size_t hko_uniform_packed_bytes(size_t rows, size_t cols, int bits, size_t group);
int hko_uniform_pack(const float* w, size_t rows, size_t cols, int bits, size_t group, uint16_t* scales,
                     uint8_t* codes);
int hko_uniform_decode(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols, int bits,
                       size_t group, float* out);
int hko_uniform_matvec(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols, int bits,
                       size_t group, const float* x, float* y);
int hko_uniform_matvec_f64(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols, int bits,
                           size_t group, const double* x, double* y);
/* y = L (R x): L [rows x rank], R [rank x cols], both uniform factors of one bits/group. */
int hko_hgravs01_matvec(const uint16_t* ls, const uint8_t* lc, size_t rows, size_t rank, const uint16_t* rs,
                        const uint8_t* rc, size_t cols, int bits, size_t group, const float* x, float* y);

/* HGRAVR02 rice_q1_rms (q80_mixed_decode.rs:260-527). */
uint32_t hko_best_rice_k(const uint32_t* v, size_t n);
size_t hko_rice_bytes(const uint32_t* v, size_t n, uint32_t k);
void hko_rice_pack(const uint32_t* v, size_t n, uint32_t k, uint8_t* out);
int hko_rice_unpack(const uint8_t* p, size_t len, size_t count, uint32_t k, uint32_t* out);
int hko_rice_expand(uint32_t first, const uint8_t* rice, size_t rice_len, uint32_t k, size_t count,
                    uint32_t* indices);
int hko_rice_row_ptr(const uint32_t* indices, size_t count, size_t rows, size_t cols, uint32_t* row_ptr);
size_t hko_rice_q1_count(size_t n, double ratio);
int hko_rice_q1_pack(const float* w, size_t rows, size_t cols, double ratio, uint16_t* bin_scales,
                     uint8_t* bin_signs, uint32_t* indices, uint8_t* res_signs, uint16_t* res_scale,
                     uint32_t* first, uint32_t* rice_k, uint8_t* rice, size_t rice_cap, size_t* rice_len);
int hko_rice_q1_apply(const uint32_t* indices, const uint8_t* res_signs, size_t count, uint16_t res_scale,
                      size_t rows, size_t cols, const float* x, float* y);
int hko_rice_q1_matvec(const uint16_t* bin_scales, const uint8_t* bin_signs, size_t rows, size_t cols,
                       const uint32_t* indices, const uint8_t* res_signs, size_t count, uint16_t res_scale,
                       const float* x, float* y);
int hko_rice_q1_matvec_f64(const uint16_t* bin_scales, const uint8_t* bin_signs, size_t rows, size_t cols,
                           const uint32_t* indices, const uint8_t* res_signs, size_t count, uint16_t res_scale,
                           const double* x, double* y);

/* ---- mixed <=1.5 BPW, per 128-group binary|Q2 (build-defined canonical stream):
 *   tags  u8[ceil(groups/8)]  LSB-first over flat group index, bit 1 = binary
 *   bin_scales f16[n_bin]     bin_signs u8[n_bin*16]      (binary groups in flat order)
 *   q2_scales  f16[2*n_q2]    q2_codes  u8[n_q2*32]       (Q2 groups in flat order)
 * Requires cols % 128 == 0. ---- */
typedef struct hko_mixed {
    size_t rows, cols;
    size_t n_bin, n_q2;
    uint8_t* tags;
    uint16_t* bin_scales;
    uint8_t* bin_signs;
    uint16_t* q2_scales;
    uint8_t* q2_codes;
} hko_mixed;
/* Pack with the per-group selector: is_binary[g] (flat group index) != 0 -> binary. */
int hko_mixed_pack(const float* w, size_t rows, size_t cols, const uint8_t* is_binary,
                   hko_mixed* out);
void hko_mixed_free(hko_mixed* m);
int hko_mixed_decode(const hko_mixed* m, float* out);
int hko_mixed_matvec(const hko_mixed* m, const float* x, float* y);
int hko_mixed_matvec_f64(const hko_mixed* m, const double* x, double* y);

/* ---- dense f32 gemv: gemv_f32 (src/kernels/mod.rs:299-311) ---- */
void hko_gemv_f32(const float* w, size_t rows, size_t cols, const float* x, float* y);

/* ---- router / activations ---- */
/* source_qwen80_topk_router (src/model/qwen80_complete_runtime.rs:5970-6025)
 * generalised to n_experts/top_k; tie_eps = HAWKING_DS_ROUTE_TIE_EPS (src/moe.rs:8-14).
 * Runs Qwen80RouteSelection::validate (qwen80_complete_runtime.rs:1522-1542). */
int hko_router_softmax_topk(const float* logits, size_t n_experts, size_t top_k,
                            float tie_eps, int32_t* ids, float* weights);
/* topk_softmax_batch (src/kernels/mod.rs:342-374): softmax_inplace (mul by 1/sum),
 * mask-and-pick, no renorm.  Used by the ported tie fixtures. */
void hko_topk_softmax_batch(const float* logits, size_t n_tokens, size_t n_experts,
                            size_t top_k, int32_t* ids, float* weights);
/* noaux_tc router (src/gravity_glm.rs:447-500) on given logits. */
int hko_router_noaux_tc(const float* logits, const float* bias, size_t n_experts,
                        size_t n_group, size_t topk_group, size_t top_k, int norm_topk_prob,
                        float routed_scaling_factor, int32_t* ids, float* weights);
/* topk_desc (src/gravity_glm.rs:230-240): stable descending, ties -> lower index. */
void hko_topk_desc(const float* values, size_t n, size_t k, int32_t* out);
/* source_qwen80_residual_rms_norm (qwen80_complete_runtime.rs:6778-6797), eps given. */
int hko_rmsnorm_1p(const float* x, const float* w, size_t n, float eps, float* out);
int hko_argmax_greedy(const float* logits, size_t n_valid, int32_t* token);
int hko_terminal_greedy(const float* hidden, const float* norm_w, size_t hidden_n, float eps, const uint16_t* scales,
                        const uint8_t* codes, size_t vocab, size_t n_valid, float* logits, int32_t* token);
/* silu_mul (src/kernels/mod.rs:24-31). */
void hko_silu_mul(const float* gate, const float* up, size_t n, float* out);

/* ---- MoE layer (moe_suffix, qwen80_uniform_q4_hybrid_decode.rs:2615-2757) ----
 * One organ is either Q4 (kind 0) or mixed (kind 2). */
typedef struct hko_organ {
    int kind;          /* 0 = Q4, 1 = binary, 2 = mixed, 3 = uniform q8 G64 (HGRAVU01),
                          4 = low-rank 3-bit G64 factors (HGRAVS01), 5 = binary + Rice residual (HGRAVR02) */
    int group;         /* Q4 group size; 128 for binary; 64 for the uniform factors */
    size_t rows, cols;
    const uint16_t* scales;   /* Q4 / binary / q8 / HGRAVS01 left factor / HGRAVR02 base */
    const uint8_t* codes;     /* codes or binary signs, as for scales */
    const hko_mixed* mixed;   /* kind 2 */
    size_t rank;              /* kind 4: left is rows x rank, right rank x cols */
    const uint16_t* r_scales; /* kind 4: right factor */
    const uint8_t* r_codes;
    const uint32_t* res_indices; /* kind 5: outlier flat indices (expanded), signs, count, f16 scale */
    const uint8_t* res_signs;
    size_t res_count;
    uint16_t res_scale;
} hko_organ;
int hko_organ_matvec(const hko_organ* o, const float* x, float* y);
int hko_organ_matvec_f64(const hko_organ* o, const double* x, double* y);
/* source_qwen80_mlp (qwen80_complete_runtime.rs:6074-6107). act may be NULL. */
int hko_mlp(const hko_organ* gate, const hko_organ* up, const hko_organ* down,
            const float* x, float* act, float* out);

typedef struct hko_moe_layer {
    size_t hidden, inter, n_experts, top_k;
    float eps;
    const float* norm_w;        /* [hidden], applied as (1 + w) */
    const float* router_w;      /* [n_experts x hidden] f32 */
    const float* shared_gate_w; /* [hidden] or NULL (no sigmoid gate: weight 1) */
    const hko_organ* experts;   /* [n_experts * 3]: gate, up, down per expert */
    const hko_organ* shared;    /* [3] or NULL */
    float tie_eps;              /* router tie window (route_tie_epsilon, src/moe.rs:8-14); 0 = strict */
} hko_moe_layer;
/* Full moe_suffix: out = h + sum_r w_r*mlp_r(xn) (route order) + g*shared(xn).
 * ids/weights/xn may be NULL. */
int hko_moe_layer_forward(const hko_moe_layer* L, const float* h, float* out,
                          int32_t* ids, float* weights, float* xn_out, float* logits_out);
/* FP64 authority for one layer given the route (ids/weights from the f32 path). */
int hko_moe_layer_forward_f64(const hko_moe_layer* L, const double* h, const int32_t* ids,
                              const float* weights, double* out);

/* ---- noaux_tc MoE block (src/gravity_glm.rs:447-600, routed_moe) ---- */
typedef struct hko_noaux_moe {
    size_t hidden, n_experts, top_k, n_group, topk_group;
    int norm_topk_prob;
    float routed_scaling_factor;
    const float* router_w;    /* [n_experts x hidden] f32 */
    const float* bias;        /* [n_experts] e_score_correction_bias */
    const hko_organ* experts; /* [n_experts * 3]: gate, up, down per expert */
    const hko_organ* shared;  /* [3] or NULL */
} hko_noaux_moe;
/* One token: out = sum over the routed experts in ascending id of w_e*mlp_e(x),
 * then + mlp_shared(x) (weight 1).  x is the block input (no norm, no residual).
 * ids/weights (top_k, route order) and logits may be NULL. */
int hko_noaux_moe_forward(const hko_noaux_moe* M, const float* x, float* out, int32_t* ids, float* weights,
                          float* logits);
/* FP64 authority for one token given its route ids: sigmoid scores, renorm and
 * scaling, every MLP and the combine in f64. */
int hko_noaux_moe_forward_f64(const hko_noaux_moe* M, const double* x, const int32_t* ids, double* out);

/* ---- numeric contract (src/numeric_parity.rs:79-118, 323-358) ---- */
double hko_relative_l2_f32(const float* candidate, const float* reference, size_t n);
double hko_relative_l2_f64ref(const float* candidate, const double* reference, size_t n);

#ifdef __cplusplus
}
#endif
#endif
