/*
 * hk_oracle.c -- CPU oracle for the quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see hk_oracle.h).  Plain-C restatement of the
 * reference's serial CPU functions, each citing the Rust function it follows
 * (paths relative to crates/hawking-core/src/ unless stated).  Compile with
 * -O2 -ffp-contract=off and without -ffast-math: every f32 operation below is
 * a separate IEEE round-to-nearest-even step, in the reference's order.
 */
#include "hk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* IEEE binary16                                                             */
/* ------------------------------------------------------------------------ */

/* f32 -> f16, round to nearest even (what half::f16::from_f32 does). */
uint16_t hko_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) {
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t half_m = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t half_m = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t h = sign | ((uint32_t)e << 10) | half_m;
    if (rem > 0x1000u || (rem == 0x1000u && (half_m & 1u))) h++;
    return (uint16_t)h;
}

float hko_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)bits >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)bits & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        if (man == 0) {
            out = sign;
        } else {
            /* subnormal: normalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            out = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1Fu) {
        out = sign | 0x7F800000u | (man << 13);
    } else {
        out = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

static float signum_f32(float v) { return signbit(v) ? -1.0f : 1.0f; }

/* rint_ties_even, qwen_complete_binary/qwen80_uniform_q4.rs:170-188, literally. */
float hko_rint_ties_even(float value) {
    if (!isfinite(value)) return value;
    float truncated = truncf(value);
    float fraction = value - truncated;
    float abs_fraction = fabsf(fraction);
    if (abs_fraction < 0.5f) return truncated;
    if (abs_fraction > 0.5f) return truncated + signum_f32(value);
    if (((int64_t)truncated) % 2 == 0) return truncated;
    return truncated + signum_f32(value);
}

/* ------------------------------------------------------------------------ */
/* Reference generators: q80_mixed_decode.rs:631-647                         */
/* ------------------------------------------------------------------------ */

void hko_deterministic_matrix(size_t rows, size_t cols, uint32_t seed, float* out) {
    for (size_t i = 0; i < rows * cols; ++i) {
        float phase = (float)((uint32_t)i * 1103515245u + seed);
        out[i] = (fmodf(phase, 251.0f) - 125.0f) / 251.0f;
    }
}

void hko_deterministic_input(size_t cols, float* out) {
    for (size_t i = 0; i < cols; ++i) {
        float phase = (float)(i % 17);
        out[i] = sinf(phase * 0.07f - 0.5f);
    }
}

/* ------------------------------------------------------------------------ */
/* Synthetic generator (build-defined; the GPU generator must match bits).   */
/* ------------------------------------------------------------------------ */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t hko_stream_key(uint64_t seed, uint64_t stream) {
    return mix64(mix64(seed ^ 0x6A09E667F3BCC909ull) ^ stream);
}

static uint64_t stream_word(uint64_t key, uint64_t ctr) {
    return mix64(key + (ctr + 1u) * 0x9E3779B97F4A7C15ull);
}

/* Irwin-Hall(12) - 6 from twelve 16-bit uniforms (u + 1/2) / 2^16: the sum
 * S = sum(2u+1) - 12*2^16 is an exact integer, z = S / 2^17 is exact in f32,
 * and the only rounding step is the final multiply by sigma. */
float hko_normal(uint64_t key, uint64_t index, float sigma) {
    int32_t s = 0;
    for (int w = 0; w < 3; ++w) {
        uint64_t v = stream_word(key, index * 3u + (uint64_t)w);
        for (int j = 0; j < 4; ++j) s += (int32_t)((v >> (16 * j)) & 0xFFFFu);
    }
    int32_t S = 2 * s + 12 - 786432;
    float z = (float)S * (1.0f / 131072.0f);
    return z * sigma;
}

void hko_fill_normal(uint64_t key, size_t count, float sigma, float* out) {
    for (size_t i = 0; i < count; ++i) out[i] = hko_normal(key, (uint64_t)i, sigma);
}

void hko_fill_normal_from(uint64_t key, uint64_t first, size_t count, float sigma, float* out) {
    for (size_t i = 0; i < count; ++i) out[i] = hko_normal(key, first + (uint64_t)i, sigma);
}

/* p(binary) = 0.7: threshold floor(0.7 * 2^32). */
int hko_mixed_coin(uint64_t coin_key, uint64_t group) {
    uint32_t u = (uint32_t)(stream_word(coin_key, group) >> 32);
    return u < 3006477107u;
}

void hko_fill_coins(uint64_t coin_key, size_t groups, uint8_t* out) {
    for (size_t g = 0; g < groups; ++g) out[g] = (uint8_t)hko_mixed_coin(coin_key, (uint64_t)g);
}

/* ------------------------------------------------------------------------ */
/* Q4 uniform                                                                */
/* ------------------------------------------------------------------------ */

static int q4_group_ok(int group) { return group == 32 || group == 64 || group == 128; }

static int all_finite(const float* v, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) return 0;
    return 1;
}

/* pack_uniform_q4_group64, qwen80_uniform_q4.rs:190-278 (flat groups of G). */
int hko_q4_pack(const float* w, size_t rows, size_t cols, int group, uint16_t* scales,
                uint8_t* codes) {
    if (!q4_group_ok(group)) return HKO_E_UNSUPPORTED;
    if (rows == 0 || cols == 0 || cols % (size_t)group) return HKO_E_GEOMETRY;
    size_t elements = rows * cols;
    if (!all_finite(w, elements)) return HKO_E_NONFINITE;
    size_t groups = elements / (size_t)group;
    size_t cb = (size_t)group / 2;
    memset(codes, 0, groups * cb);
    for (size_t g = 0; g < groups; ++g) {
        const float* v = w + g * (size_t)group;
        float max_abs = 0.0f;
        for (int i = 0; i < group; ++i) max_abs = fmaxf(max_abs, fabsf(v[i]));
        uint16_t scale = hko_f32_to_f16(max_abs / 7.0f);
        if ((scale & 0x7C00u) == 0x7C00u) return HKO_E_NONFINITE;
        float rs = hko_f16_to_f32(scale);
        scales[g] = scale;
        for (int local = 0; local < group; ++local) {
            int32_t q;
            if (rs == 0.0f) {
                q = 0;
            } else {
                float r = hko_rint_ties_even(v[local] / rs);
                if (r < -8.0f) r = -8.0f;
                if (r > 7.0f) r = 7.0f;
                q = (int32_t)r;
            }
            uint8_t code = (uint8_t)(q + 8);
            if ((local & 1) == 0)
                codes[g * cb + (size_t)local / 2] |= code;
            else
                codes[g * cb + (size_t)local / 2] |= (uint8_t)(code << 4);
        }
    }
    return HKO_OK;
}

/* decode_uniform_q4_group64, qwen80_uniform_q4.rs:325-346. */
int hko_q4_decode(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols,
                  int group, float* out) {
    if (!q4_group_ok(group)) return HKO_E_UNSUPPORTED;
    if (cols % (size_t)group) return HKO_E_GEOMETRY;
    size_t elements = rows * cols;
    size_t cb = (size_t)group / 2;
    for (size_t e = 0; e < elements; ++e) {
        size_t g = e / (size_t)group, local = e % (size_t)group;
        float scale = hko_f16_to_f32(scales[g]);
        uint8_t packed = codes[g * cb + local / 2];
        uint8_t nibble = (local & 1) == 0 ? (packed & 0x0F) : (packed >> 4);
        out[e] = (float)((int32_t)nibble - 8) * scale;
    }
    return HKO_OK;
}

/* Qwen80Q4PackedTensor::matvec, qwen80_uniform_q4_hybrid_decode.rs:957-1036:
 * per row, groups left to right, (even, odd) pairs, sum += (q*scale)*x. */
int hko_q4_matvec(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols,
                  int group, const float* x, float* y) {
    if (!q4_group_ok(group)) return HKO_E_UNSUPPORTED;
    if (cols % (size_t)group) return HKO_E_GEOMETRY;
    if (!all_finite(x, cols)) return HKO_E_NONFINITE;
    size_t gpr = cols / (size_t)group, cb = (size_t)group / 2;
    for (size_t row = 0; row < rows; ++row) {
        float sum = 0.0f;
        for (size_t g = 0; g < gpr; ++g) {
            size_t col0 = g * (size_t)group;
            size_t gi = row * gpr + g;
            float scale = hko_f16_to_f32(scales[gi]);
            const uint8_t* c = codes + gi * cb;
            for (size_t local = 0; local + 1 < (size_t)group; local += 2) {
                uint8_t packed = c[local / 2];
                int32_t q0 = (int32_t)(packed & 0x0F) - 8;
                int32_t q1 = (int32_t)(packed >> 4) - 8;
                sum += (float)q0 * scale * x[col0 + local];
                sum += (float)q1 * scale * x[col0 + local + 1];
            }
        }
        if (!isfinite(sum)) return HKO_E_NONFINITE;
        y[row] = sum;
    }
    return HKO_OK;
}

int hko_q4_matvec_f64(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols,
                      int group, const double* x, double* y) {
    if (!q4_group_ok(group)) return HKO_E_UNSUPPORTED;
    if (cols % (size_t)group) return HKO_E_GEOMETRY;
    size_t gpr = cols / (size_t)group, cb = (size_t)group / 2;
    for (size_t row = 0; row < rows; ++row) {
        double sum = 0.0;
        for (size_t g = 0; g < gpr; ++g) {
            size_t gi = row * gpr + g;
            double scale = (double)hko_f16_to_f32(scales[gi]);
            const uint8_t* c = codes + gi * cb;
            for (size_t local = 0; local < (size_t)group; ++local) {
                uint8_t packed = c[local / 2];
                int32_t q = (int32_t)((local & 1) ? (packed >> 4) : (packed & 0x0F)) - 8;
                sum += (double)q * scale * x[g * (size_t)group + local];
            }
        }
        y[row] = sum;
    }
    return HKO_OK;
}

/* dequant_q4_0, src/quant.rs:473-498: lo nibble -> j, hi nibble -> j+16. */
int hko_q4_0_dequant(const uint8_t* blocks, size_t elements, float* out) {
    if (elements % 32) return HKO_E_GEOMETRY;
    for (size_t b = 0; b < elements / 32; ++b) {
        const uint8_t* blk = blocks + b * 18;
        float d = hko_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 16; ++j) {
            int32_t lo = (int32_t)(blk[2 + j] & 0x0F) - 8;
            int32_t hi = (int32_t)((blk[2 + j] >> 4) & 0x0F) - 8;
            out[b * 32 + (size_t)j] = d * (float)lo;
            out[b * 32 + (size_t)j + 16] = d * (float)hi;
        }
    }
    return HKO_OK;
}

/* ------------------------------------------------------------------------ */
/* Binary sign plane                                                         */
/* ------------------------------------------------------------------------ */

/* One group of pack_binary_group (q80_mixed_decode.rs:185-230): mean |w| in
 * f64, then f64 -> f32 -> f16 (two roundings); sign bit = (w >= 0). */
static uint16_t bin_pack_group(const float* v, int group, uint8_t* signs, size_t bit0) {
    double sum_abs = 0.0;
    for (int i = 0; i < group; ++i) {
        sum_abs += (double)fabsf(v[i]);
        if (v[i] >= 0.0f) signs[(bit0 + (size_t)i) >> 3] |= (uint8_t)(1u << ((bit0 + (size_t)i) & 7u));
    }
    double mean = sum_abs / (double)group;
    return hko_f32_to_f16((float)mean);
}

int hko_bin_pack(const float* w, size_t rows, size_t cols, int group, uint16_t* scales,
                 uint8_t* signs) {
    if (rows == 0 || cols == 0 || group <= 0) return HKO_E_GEOMETRY;
    if (cols % (size_t)group) return HKO_E_GEOMETRY;
    if (!all_finite(w, rows * cols)) return HKO_E_NONFINITE;
    size_t gpr = cols / (size_t)group;
    memset(signs, 0, (rows * cols + 7) / 8);
    for (size_t row = 0; row < rows; ++row)
        for (size_t g = 0; g < gpr; ++g) {
            size_t start = row * cols + g * (size_t)group;
            scales[row * gpr + g] = bin_pack_group(w + start, group, signs, start);
        }
    return HKO_OK;
}

/* binary_group_weight, q80_mixed_decode.rs:232-243. */
static float bin_weight(const uint16_t* scales, const uint8_t* signs, size_t cols, int group,
                        size_t row, size_t col) {
    size_t flat = row * cols + col;
    float scale = hko_f16_to_f32(scales[row * (cols / (size_t)group) + col / (size_t)group]);
    int positive = (signs[flat >> 3] >> (flat & 7u)) & 1u;
    return positive ? scale : -scale;
}

int hko_bin_decode(const uint16_t* scales, const uint8_t* signs, size_t rows, size_t cols,
                   int group, float* out) {
    if (group <= 0 || cols % (size_t)group) return HKO_E_GEOMETRY;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] = bin_weight(scales, signs, cols, group, r, c);
    return HKO_OK;
}

/* binary_group_matvec_f32, q80_mixed_decode.rs:245-257: serial sum += w*x. */
int hko_bin_matvec(const uint16_t* scales, const uint8_t* signs, size_t rows, size_t cols,
                   int group, const float* x, float* y) {
    if (group <= 0 || cols % (size_t)group) return HKO_E_GEOMETRY;
    if (!all_finite(x, cols)) return HKO_E_NONFINITE;
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) sum += bin_weight(scales, signs, cols, group, r, c) * x[c];
        y[r] = sum;
    }
    return HKO_OK;
}

int hko_bin_matvec_f64(const uint16_t* scales, const uint8_t* signs, size_t rows, size_t cols,
                       int group, const double* x, double* y) {
    if (group <= 0 || cols % (size_t)group) return HKO_E_GEOMETRY;
    for (size_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (size_t c = 0; c < cols; ++c)
            sum += (double)bin_weight(scales, signs, cols, group, r, c) * x[c];
        y[r] = sum;
    }
    return HKO_OK;
}

/* ------------------------------------------------------------------------ */
/* Q2 stage (group 64)                                                       */
/* ------------------------------------------------------------------------ */

/* One 64-group of _additive_residual_codec's base stage
 * (lab/operators/ascension_dual_gravity_worker.py:898-911): scale =
 * f16(max|w| / 1.5) in f32; denominator = scale or 1; code =
 * clip(rint(w/denominator + 1.5), 0, 3); codes packed 2 bits LSB-first. */
static uint16_t q2_pack_group(const float* v, uint8_t* codes, size_t elem0) {
    float max_abs = 0.0f;
    for (int i = 0; i < 64; ++i) max_abs = fmaxf(max_abs, fabsf(v[i]));
    uint16_t scale = hko_f32_to_f16(max_abs / 1.5f);
    float sf = hko_f16_to_f32(scale);
    float denom = sf > 0.0f ? sf : 1.0f;
    for (int i = 0; i < 64; ++i) {
        float n = v[i] / denom;
        float r = hko_rint_ties_even(n + 1.5f);
        if (r < 0.0f) r = 0.0f;
        if (r > 3.0f) r = 3.0f;
        uint32_t code = (uint32_t)r;
        size_t e = elem0 + (size_t)i;
        codes[e >> 2] |= (uint8_t)(code << (2u * (e & 3u)));
    }
    return scale;
}

static float q2_level(uint32_t code, float sf) { return ((float)code - 1.5f) * sf; }

int hko_q2_pack(const float* w, size_t count, uint16_t* scales, uint8_t* codes) {
    if (count == 0 || count % 64) return HKO_E_GEOMETRY;
    if (!all_finite(w, count)) return HKO_E_NONFINITE;
    memset(codes, 0, count / 4);
    for (size_t g = 0; g < count / 64; ++g) scales[g] = q2_pack_group(w + g * 64, codes, g * 64);
    return HKO_OK;
}

int hko_q2_decode(const uint16_t* scales, const uint8_t* codes, size_t count, float* out) {
    if (count % 64) return HKO_E_GEOMETRY;
    for (size_t e = 0; e < count; ++e) {
        uint32_t code = (codes[e >> 2] >> (2u * (e & 3u))) & 3u;
        out[e] = q2_level(code, hko_f16_to_f32(scales[e / 64]));
    }
    return HKO_OK;
}

/* ------------------------------------------------------------------------ */
/* Uniform factor codec (HGRAVU01 q8 G64, HGRAVS01 factors)                  */
/* ------------------------------------------------------------------------ */

/* pack_unsigned / packed_byte_count (q80_mixed_decode.rs:83-92,149-183):
 * codes of `bits` bits, LSB-first bitstream. */
size_t hko_uniform_packed_bytes(size_t rows, size_t cols, int bits, size_t group) {
    if (bits < 1 || bits > 8 || group == 0) return 0;
    size_t elements = rows * cols, groups = (elements + group - 1) / group;
    return (groups * group * (size_t)bits + 7) / 8;
}

static void put_unsigned(uint8_t* codes, size_t element, int bits, uint32_t value) {
    size_t bit0 = element * (size_t)bits;
    for (int b = 0; b < bits; ++b) {
        size_t bi = bit0 + (size_t)b;
        if ((value >> b) & 1u) codes[bi >> 3] |= (uint8_t)(1u << (bi & 7u));
    }
}

/* extract_unsigned (q80_mixed_decode.rs:579-589). */
static uint32_t get_unsigned(const uint8_t* codes, size_t element, int bits) {
    size_t bit0 = element * (size_t)bits;
    uint32_t value = 0;
    for (int b = 0; b < bits; ++b) {
        size_t bi = bit0 + (size_t)b;
        value |= (uint32_t)((codes[bi >> 3] >> (bi & 7u)) & 1u) << b;
    }
    return value;
}

/* pack_uniform_factor (q80_mixed_decode.rs:529-577): groups over the flat
 * elements, the last possibly partial (missing values pack as 0); bound =
 * 2^(bits-1) - 1; scale = f16(max|w| / bound) (f32 divide); the quantizer
 * divides by the f32 scale before rounding (1 when it is 0) and rounds half
 * away from zero (Rust f32::round); code = q + bound. */
int hko_uniform_pack(const float* w, size_t rows, size_t cols, int bits, size_t group, uint16_t* scales,
                     uint8_t* codes) {
    if (bits < 2 || bits > 8 || group == 0 || rows == 0 || cols == 0) return HKO_E_GEOMETRY;
    size_t elements = rows * cols;
    if (!all_finite(w, elements)) return HKO_E_NONFINITE;
    size_t groups = (elements + group - 1) / group;
    uint32_t bound = (1u << (bits - 1)) - 1u;
    memset(codes, 0, hko_uniform_packed_bytes(rows, cols, bits, group));
    for (size_t g = 0; g < groups; ++g) {
        size_t start = g * group, end = start + group < elements ? start + group : elements;
        float max_abs = 0.0f;
        for (size_t e = start; e < end; ++e) max_abs = fmaxf(max_abs, fabsf(w[e]));
        float scale = max_abs / (float)(bound ? bound : 1u);
        scales[g] = hko_f32_to_f16(scale);
        float denom = scale > 0.0f ? scale : 1.0f;
        for (size_t i = 0; i < group; ++i) {
            float value = start + i < elements ? w[start + i] : 0.0f;
            float q = roundf(value / denom);
            if (q < -(float)bound) q = -(float)bound;
            if (q > (float)bound) q = (float)bound;
            put_unsigned(codes, start + i, bits, (uint32_t)((int32_t)q + (int32_t)bound));
        }
    }
    return HKO_OK;
}

/* uniform_factor_value (q80_mixed_decode.rs:591-598): (code - bound) * f32(scale). */
static float uniform_value(const uint16_t* scales, const uint8_t* codes, size_t element, int bits, size_t group) {
    int32_t bound = (int32_t)((1u << (bits - 1)) - 1u);
    float scale = hko_f16_to_f32(scales[element / group]);
    return (float)((int32_t)get_unsigned(codes, element, bits) - bound) * scale;
}

int hko_uniform_decode(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols, int bits,
                       size_t group, float* out) {
    if (bits < 2 || bits > 8 || group == 0) return HKO_E_GEOMETRY;
    for (size_t e = 0; e < rows * cols; ++e) out[e] = uniform_value(scales, codes, e, bits, group);
    return HKO_OK;
}

/* uniform_factor_matvec_f32 (q80_mixed_decode.rs:600-612): per row, serial
 * f32 sum += value * x over the columns; x must be finite. */
int hko_uniform_matvec(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols, int bits,
                       size_t group, const float* x, float* y) {
    if (bits < 2 || bits > 8 || group == 0) return HKO_E_GEOMETRY;
    if (!all_finite(x, cols)) return HKO_E_NONFINITE;
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) sum += uniform_value(scales, codes, r * cols + c, bits, group) * x[c];
        y[r] = sum;
    }
    return HKO_OK;
}

int hko_uniform_matvec_f64(const uint16_t* scales, const uint8_t* codes, size_t rows, size_t cols, int bits,
                           size_t group, const double* x, double* y) {
    if (bits < 2 || bits > 8 || group == 0) return HKO_E_GEOMETRY;
    for (size_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (size_t c = 0; c < cols; ++c) sum += (double)uniform_value(scales, codes, r * cols + c, bits, group) * x[c];
        y[r] = sum;
    }
    return HKO_OK;
}

/* hgravs01_two_stage_matvec_f32 (q80_mixed_decode.rs:614-629): mid = R x, y = L mid. */
int hko_hgravs01_matvec(const uint16_t* ls, const uint8_t* lc, size_t rows, size_t rank, const uint16_t* rs,
                        const uint8_t* rc, size_t cols, int bits, size_t group, const float* x, float* y) {
    float* mid = (float*)malloc(rank * sizeof(float));
    if (!mid) return HKO_E_INVALID_ARG;
    int rc0 = hko_uniform_matvec(rs, rc, rank, cols, bits, group, x, mid);
    if (rc0 == HKO_OK) rc0 = hko_uniform_matvec(ls, lc, rows, rank, bits, group, mid, y);
    free(mid);
    return rc0;
}

/* ------------------------------------------------------------------------ */
/* HGRAVR02: binary base + Rice-coded 1-bit residual (rice_q1_rms)           */
/* ------------------------------------------------------------------------ */

/* best_rice_k (q80_mixed_decode.rs:314-333): the k in 0..15 minimising
 * sum(v >> k) + n (1 + k), the first on ties; 0 for no values. */
uint32_t hko_best_rice_k(const uint32_t* v, size_t n) {
    if (n == 0) return 0;
    uint32_t best_k = 0;
    uint64_t best_bits = UINT64_MAX;
    for (uint32_t k = 0; k < 16; ++k) {
        uint64_t q = 0;
        for (size_t i = 0; i < n; ++i) q += (uint64_t)(v[i] >> k);
        uint64_t bits = q + (uint64_t)n * (1u + k);
        if (bits < best_bits) {
            best_bits = bits;
            best_k = k;
        }
    }
    return best_k;
}

/* Bytes of pack_rice's output: per value (v >> k) ones, a zero, k LSBs. */
size_t hko_rice_bytes(const uint32_t* v, size_t n, uint32_t k) {
    uint64_t bits = 0;
    for (size_t i = 0; i < n; ++i) bits += (uint64_t)(v[i] >> k) + 1u + k;
    return (size_t)((bits + 7) / 8);
}

static void put_bit(uint8_t* out, uint64_t* pos, uint32_t bit) {
    if (bit) out[*pos >> 3] |= (uint8_t)(1u << (*pos & 7u));
    ++*pos;
}

/* pack_rice / BitWriter (q80_mixed_decode.rs:260-346): LSB-first bits; the
 * last byte is zero-padded.  out holds hko_rice_bytes(v, n, k) bytes. */
void hko_rice_pack(const uint32_t* v, size_t n, uint32_t k, uint8_t* out) {
    memset(out, 0, hko_rice_bytes(v, n, k));
    uint64_t pos = 0;
    for (size_t i = 0; i < n; ++i) {
        for (uint32_t q = v[i] >> k; q; --q) put_bit(out, &pos, 1);
        put_bit(out, &pos, 0);
        for (uint32_t b = 0; b < k; ++b) put_bit(out, &pos, (v[i] >> b) & 1u);
    }
}

/* unpack_rice (q80_mixed_decode.rs:348-381): reading past `len` bytes and a
 * quotient above u32 are errors. */
int hko_rice_unpack(const uint8_t* p, size_t len, size_t count, uint32_t k, uint32_t* out) {
    uint64_t pos = 0, end = (uint64_t)len * 8u;
    for (size_t i = 0; i < count; ++i) {
        uint64_t q = 0;
        for (;;) {
            if (pos >= end) return HKO_E_GEOMETRY;
            uint32_t bit = (p[pos >> 3] >> (pos & 7u)) & 1u;
            ++pos;
            if (!bit) break;
            if (++q > UINT32_MAX) return HKO_E_GEOMETRY;
        }
        uint32_t rem = 0;
        for (uint32_t b = 0; b < k; ++b) {
            if (pos >= end) return HKO_E_GEOMETRY;
            rem |= (uint32_t)((p[pos >> 3] >> (pos & 7u)) & 1u) << b;
            ++pos;
        }
        out[i] = (uint32_t)(q << k) | rem;  /* the reference's u32 shift */
    }
    return HKO_OK;
}

/* expand_rice_indices (q80_mixed_decode.rs:486-507): first, then running
 * sums of the diffs; an index above u32 is an error. */
int hko_rice_expand(uint32_t first, const uint8_t* rice, size_t rice_len, uint32_t k, size_t count,
                    uint32_t* indices) {
    if (count == 0) return HKO_E_GEOMETRY;
    indices[0] = first;
    if (count == 1) return HKO_OK;
    int rc = hko_rice_unpack(rice, rice_len, count - 1, k, indices + 1);
    if (rc) return rc;
    uint64_t acc = first;
    for (size_t i = 1; i < count; ++i) {
        acc += indices[i];
        if (acc > UINT32_MAX) return HKO_E_GEOMETRY;
        indices[i] = (uint32_t)acc;
    }
    return HKO_OK;
}

/* rice_q1_row_ptr (q80_mixed_decode.rs:462-484): CSR row pointers. */
int hko_rice_row_ptr(const uint32_t* indices, size_t count, size_t rows, size_t cols, uint32_t* row_ptr) {
    if (cols == 0) return HKO_E_GEOMETRY;
    memset(row_ptr, 0, (rows + 1) * sizeof(uint32_t));
    for (size_t i = 0; i < count; ++i) {
        size_t row = indices[i] / cols;
        if (row >= rows) return HKO_E_GEOMETRY;
        row_ptr[row + 1] += 1;
    }
    for (size_t r = 0; r < rows; ++r) row_ptr[r + 1] += row_ptr[r];
    return HKO_OK;
}

size_t hko_rice_q1_count(size_t n, double ratio) {
    size_t count = (size_t)ceil((double)n * ratio);
    if (count < 1) count = 1;
    if (count > n) count = n;
    return count;
}

/* qsort's comparator reads the magnitudes through this pointer; one per
 * thread, so packs on several threads at once do not see each other's. */
static _Thread_local const float* g_sort_abs;
static int by_abs_desc_then_index(const void* a, const void* b) {
    uint32_t i = *(const uint32_t*)a, j = *(const uint32_t*)b;
    float x = g_sort_abs[i], y = g_sort_abs[j];
    if (x > y) return -1;
    if (x < y) return 1;
    return i < j ? -1 : (i > j ? 1 : 0);
}
static int u32_ascending(const void* a, const void* b) {
    uint32_t i = *(const uint32_t*)a, j = *(const uint32_t*)b;
    return i < j ? -1 : (i > j ? 1 : 0);
}

/* pack_binary_rice_q1 (q80_mixed_decode.rs:383-460): binary group-128 base;
 * residual = w - binary weight; the count = clamp(ceil(n ratio), 1, n) largest
 * |residual| (ties to the lower index), re-sorted by index; scale = f16 of
 * the f32 rounding of sqrt(mean of squares in f64) (1.0 when not finite or
 * <= 0); sign bit = residual >= 0; first index, then Rice(diffs) with
 * best_rice_k (no stream for one outlier).  Caller buffers: bin_scales
 * [n/128], bin_signs [n/8], indices [count], res_signs [(count+7)/8], rice
 * [rice_cap]; rice_cap >= (n + 17 count) / 8 + 1 always suffices. */
int hko_rice_q1_pack(const float* w, size_t rows, size_t cols, double ratio, uint16_t* bin_scales,
                     uint8_t* bin_signs, uint32_t* indices, uint8_t* res_signs, uint16_t* res_scale,
                     uint32_t* first, uint32_t* rice_k, uint8_t* rice, size_t rice_cap, size_t* rice_len) {
    if (!(ratio > 0.0 && ratio <= 0.1)) return HKO_E_INVALID_ARG;
    int rc = hko_bin_pack(w, rows, cols, 128, bin_scales, bin_signs);
    if (rc) return rc;
    size_t n = rows * cols, count = hko_rice_q1_count(n, ratio);
    float* res = (float*)malloc(n * sizeof(float));
    float* mag = (float*)malloc(n * sizeof(float));
    uint32_t* order = (uint32_t*)malloc(n * sizeof(uint32_t));
    uint32_t* diffs = (uint32_t*)malloc((count ? count : 1) * sizeof(uint32_t));
    if (!res || !mag || !order || !diffs) {
        free(res), free(mag), free(order), free(diffs);
        return HKO_E_INVALID_ARG;
    }
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) {
            size_t f = r * cols + c;
            res[f] = w[f] - bin_weight(bin_scales, bin_signs, cols, 128, r, c);
            mag[f] = fabsf(res[f]);
        }
    for (size_t i = 0; i < n; ++i) order[i] = (uint32_t)i;
    g_sort_abs = mag;
    qsort(order, n, sizeof(uint32_t), by_abs_desc_then_index);
    memcpy(indices, order, count * sizeof(uint32_t));
    qsort(indices, count, sizeof(uint32_t), u32_ascending);
    double sum_sq = 0.0;
    memset(res_signs, 0, (count + 7) / 8);
    for (size_t i = 0; i < count; ++i) {
        float v = res[indices[i]];
        sum_sq += (double)v * (double)v;
        if (v >= 0.0f) res_signs[i >> 3] |= (uint8_t)(1u << (i & 7u));
    }
    float scale = (float)sqrt(sum_sq / (double)count);
    if (!isfinite(scale) || scale <= 0.0f) scale = 1.0f;
    *res_scale = hko_f32_to_f16(scale);
    *first = indices[0];
    *rice_k = 0;
    *rice_len = 0;
    rc = HKO_OK;
    if (count > 1) {
        for (size_t i = 1; i < count; ++i) diffs[i - 1] = indices[i] - indices[i - 1];
        *rice_k = hko_best_rice_k(diffs, count - 1);
        *rice_len = hko_rice_bytes(diffs, count - 1, *rice_k);
        if (*rice_len > rice_cap) rc = HKO_E_GEOMETRY;
        else hko_rice_pack(diffs, count - 1, *rice_k, rice);
    }
    free(res), free(mag), free(order), free(diffs);
    return rc;
}

/* binary_rice_q1_matvec_f32 (q80_mixed_decode.rs:509-527): the serial binary
 * matvec, then y[flat / cols] += (+-scale) * x[flat % cols] in index order. */
int hko_rice_q1_matvec(const uint16_t* bin_scales, const uint8_t* bin_signs, size_t rows, size_t cols,
                       const uint32_t* indices, const uint8_t* res_signs, size_t count, uint16_t res_scale,
                       const float* x, float* y) {
    int rc = hko_bin_matvec(bin_scales, bin_signs, rows, cols, 128, x, y);
    if (rc) return rc;
    return hko_rice_q1_apply(indices, res_signs, count, res_scale, rows, cols, x, y);
}

/* The residual half of binary_rice_q1_matvec_f32 on its own: y += R x. */
int hko_rice_q1_apply(const uint32_t* indices, const uint8_t* res_signs, size_t count, uint16_t res_scale,
                      size_t rows, size_t cols, const float* x, float* y) {
    float scale = hko_f16_to_f32(res_scale);
    for (size_t i = 0; i < count; ++i) {
        size_t f = indices[i];
        if (f / cols >= rows) return HKO_E_GEOMETRY;
        float v = ((res_signs[i >> 3] >> (i & 7u)) & 1u) ? scale : -scale;
        y[f / cols] += v * x[f % cols];
    }
    return HKO_OK;
}

int hko_rice_q1_matvec_f64(const uint16_t* bin_scales, const uint8_t* bin_signs, size_t rows, size_t cols,
                           const uint32_t* indices, const uint8_t* res_signs, size_t count, uint16_t res_scale,
                           const double* x, double* y) {
    int rc = hko_bin_matvec_f64(bin_scales, bin_signs, rows, cols, 128, x, y);
    if (rc) return rc;
    double scale = (double)hko_f16_to_f32(res_scale);
    for (size_t i = 0; i < count; ++i) {
        size_t f = indices[i];
        if (f / cols >= rows) return HKO_E_GEOMETRY;
        double v = ((res_signs[i >> 3] >> (i & 7u)) & 1u) ? scale : -scale;
        y[f / cols] += v * x[f % cols];
    }
    return HKO_OK;
}

/* ------------------------------------------------------------------------ */
/* Mixed per-128-group binary | Q2                                           */
/* ------------------------------------------------------------------------ */

void hko_mixed_free(hko_mixed* m) {
    free(m->tags);
    free(m->bin_scales);
    free(m->bin_signs);
    free(m->q2_scales);
    free(m->q2_codes);
    memset(m, 0, sizeof(*m));
}

int hko_mixed_pack(const float* w, size_t rows, size_t cols, const uint8_t* is_binary,
                   hko_mixed* out) {
    memset(out, 0, sizeof(*out));
    if (rows == 0 || cols == 0 || cols % 128) return HKO_E_GEOMETRY;
    if (!all_finite(w, rows * cols)) return HKO_E_NONFINITE;
    size_t groups = rows * cols / 128;
    size_t n_bin = 0;
    for (size_t g = 0; g < groups; ++g) n_bin += is_binary[g] ? 1u : 0u;
    size_t n_q2 = groups - n_bin;
    out->rows = rows;
    out->cols = cols;
    out->n_bin = n_bin;
    out->n_q2 = n_q2;
    out->tags = (uint8_t*)calloc((groups + 7) / 8, 1);
    out->bin_scales = (uint16_t*)calloc(n_bin ? n_bin : 1, 2);
    out->bin_signs = (uint8_t*)calloc(n_bin ? n_bin * 16 : 1, 1);
    out->q2_scales = (uint16_t*)calloc(n_q2 ? n_q2 * 2 : 1, 2);
    out->q2_codes = (uint8_t*)calloc(n_q2 ? n_q2 * 32 : 1, 1);
    if (!out->tags || !out->bin_scales || !out->bin_signs || !out->q2_scales || !out->q2_codes) {
        hko_mixed_free(out);
        return HKO_E_INVALID_ARG;
    }
    size_t ib = 0, iq = 0;
    for (size_t g = 0; g < groups; ++g) {
        const float* v = w + g * 128;
        if (is_binary[g]) {
            out->tags[g >> 3] |= (uint8_t)(1u << (g & 7u));
            out->bin_scales[ib] = bin_pack_group(v, 128, out->bin_signs, ib * 128);
            ib++;
        } else {
            out->q2_scales[2 * iq] = q2_pack_group(v, out->q2_codes, iq * 128);
            out->q2_scales[2 * iq + 1] = q2_pack_group(v + 64, out->q2_codes, iq * 128 + 64);
            iq++;
        }
    }
    return HKO_OK;
}

/* Decoded weight of local element i (0..127) of the current group. */
static float mixed_weight(const hko_mixed* m, int binary, size_t ib, size_t iq, size_t i) {
    if (binary) {
        float s = hko_f16_to_f32(m->bin_scales[ib]);
        size_t bit = ib * 128 + i;
        return ((m->bin_signs[bit >> 3] >> (bit & 7u)) & 1u) ? s : -s;
    }
    size_t e = iq * 128 + i;
    uint32_t code = (m->q2_codes[e >> 2] >> (2u * (e & 3u))) & 3u;
    return q2_level(code, hko_f16_to_f32(m->q2_scales[2 * iq + i / 64]));
}

int hko_mixed_decode(const hko_mixed* m, float* out) {
    size_t groups = m->rows * m->cols / 128, ib = 0, iq = 0;
    for (size_t g = 0; g < groups; ++g) {
        int binary = (m->tags[g >> 3] >> (g & 7u)) & 1u;
        for (size_t i = 0; i < 128; ++i) out[g * 128 + i] = mixed_weight(m, binary, ib, iq, i);
        if (binary) ib++; else iq++;
    }
    return HKO_OK;
}

/* Same serial order as binary_group_matvec_f32: per row, column order, sum += w*x.
 * Each weight is mixed_weight's value; the group's f16 scales are converted
 * once per group (the conversion is exact, so the values are the same). */
int hko_mixed_matvec(const hko_mixed* m, const float* x, float* y) {
    if (!all_finite(x, m->cols)) return HKO_E_NONFINITE;
    size_t gpr = m->cols / 128, ib = 0, iq = 0;
    for (size_t r = 0; r < m->rows; ++r) {
        float sum = 0.0f;
        for (size_t gg = 0; gg < gpr; ++gg) {
            size_t g = r * gpr + gg;
            int binary = (m->tags[g >> 3] >> (g & 7u)) & 1u;
            const float* xg = x + gg * 128;
            if (binary) {
                const float s = hko_f16_to_f32(m->bin_scales[ib]);
                for (size_t i = 0; i < 128; ++i) {
                    size_t bit = ib * 128 + i;
                    float w = ((m->bin_signs[bit >> 3] >> (bit & 7u)) & 1u) ? s : -s;
                    sum += w * xg[i];
                }
                ib++;
            } else {
                const float s0 = hko_f16_to_f32(m->q2_scales[2 * iq]), s1 = hko_f16_to_f32(m->q2_scales[2 * iq + 1]);
                for (size_t i = 0; i < 128; ++i) {
                    size_t e = iq * 128 + i;
                    uint32_t code = (m->q2_codes[e >> 2] >> (2u * (e & 3u))) & 3u;
                    sum += q2_level(code, i < 64 ? s0 : s1) * xg[i];
                }
                iq++;
            }
        }
        if (!isfinite(sum)) return HKO_E_NONFINITE;
        y[r] = sum;
    }
    return HKO_OK;
}

int hko_mixed_matvec_f64(const hko_mixed* m, const double* x, double* y) {
    size_t gpr = m->cols / 128, ib = 0, iq = 0;
    for (size_t r = 0; r < m->rows; ++r) {
        double sum = 0.0;
        for (size_t gg = 0; gg < gpr; ++gg) {
            size_t g = r * gpr + gg;
            int binary = (m->tags[g >> 3] >> (g & 7u)) & 1u;
            for (size_t i = 0; i < 128; ++i)
                sum += (double)mixed_weight(m, binary, ib, iq, i) * x[gg * 128 + i];
            if (binary) ib++; else iq++;
        }
        y[r] = sum;
    }
    return HKO_OK;
}

/* ------------------------------------------------------------------------ */
/* Dense gemv, router, activations                                           */
/* ------------------------------------------------------------------------ */

/* gemv_f32, src/kernels/mod.rs:299-311. */
void hko_gemv_f32(const float* w, size_t rows, size_t cols, const float* x, float* y) {
    for (size_t r = 0; r < rows; ++r) {
        float acc = 0.0f;
        const float* row = w + r * cols;
        for (size_t c = 0; c < cols; ++c) acc += row[c] * x[c];
        y[r] = acc;
    }
}

/* source_qwen80_topk_router, qwen80_complete_runtime.rs:5970-6025. */
int hko_router_softmax_topk(const float* logits, size_t n_experts, size_t top_k, float tie_eps,
                            int32_t* ids, float* weights) {
    if (n_experts == 0 || top_k == 0 || top_k > n_experts) return HKO_E_INVALID_ARG;
    if (!all_finite(logits, n_experts)) return HKO_E_NONFINITE;
    float* p = (float*)malloc(n_experts * sizeof(float));
    if (!p) return HKO_E_INVALID_ARG;
    float maximum = -INFINITY;
    for (size_t i = 0; i < n_experts; ++i) maximum = fmaxf(maximum, logits[i]);
    for (size_t i = 0; i < n_experts; ++i) p[i] = expf(logits[i] - maximum);
    float sum = -0.0f;
    for (size_t i = 0; i < n_experts; ++i) sum += p[i];
    if (!isfinite(sum) || sum <= 0.0f) {
        free(p);
        return HKO_E_ROUTE;
    }
    for (size_t i = 0; i < n_experts; ++i) p[i] /= sum;
    for (size_t r = 0; r < top_k; ++r) {
        size_t best_index = 0;
        float best_value = -INFINITY;
        for (size_t index = 0; index < n_experts; ++index) {
            float value = p[index];
            int finite_pair = isfinite(best_value) && isfinite(value);
            int tied = tie_eps > 0.0f && finite_pair && fabsf(value - best_value) <= tie_eps;
            if ((value > best_value && !tied) || (tied && index < best_index)) {
                best_index = index;
                best_value = value;
            }
        }
        if (!isfinite(best_value) || best_value < 0.0f || best_index >= n_experts) {
            free(p);
            return HKO_E_ROUTE;
        }
        ids[r] = (int32_t)best_index;
        weights[r] = best_value;
        p[best_index] = -INFINITY;
    }
    free(p);
    float selected = -0.0f;
    for (size_t r = 0; r < top_k; ++r) selected += weights[r];
    if (!isfinite(selected) || selected <= 0.0f) return HKO_E_ROUTE;
    for (size_t r = 0; r < top_k; ++r) weights[r] /= selected;
    /* Qwen80RouteSelection::validate, qwen80_complete_runtime.rs:1522-1542. */
    float total = -0.0f;
    for (size_t r = 0; r < top_k; ++r) {
        for (size_t q = 0; q < r; ++q)
            if (ids[q] == ids[r]) return HKO_E_ROUTE;
        if (!isfinite(weights[r]) || weights[r] < 0.0f) return HKO_E_ROUTE;
        total += weights[r];
    }
    if (!isfinite(total) || fabsf(total - 1.0f) > 1.0e-4f) return HKO_E_ROUTE;
    return HKO_OK;
}

/* topk_softmax_batch + softmax_inplace, src/kernels/mod.rs:67-86, 342-374. */
void hko_topk_softmax_batch(const float* logits, size_t n_tokens, size_t n_experts, size_t top_k,
                            int32_t* ids, float* weights) {
    float* work = (float*)malloc(n_experts * sizeof(float));
    if (!work) return;
    for (size_t t = 0; t < n_tokens; ++t) {
        memcpy(work, logits + t * n_experts, n_experts * sizeof(float));
        float m = -INFINITY;
        for (size_t i = 0; i < n_experts; ++i)
            if (work[i] > m) m = work[i];
        float sum = 0.0f;
        for (size_t i = 0; i < n_experts; ++i) {
            work[i] = expf(work[i] - m);
            sum += work[i];
        }
        float inv = 1.0f / sum;
        for (size_t i = 0; i < n_experts; ++i) work[i] *= inv;
        for (size_t k = 0; k < top_k; ++k) {
            size_t best_idx = 0;
            float best_val = -INFINITY;
            for (size_t i = 0; i < n_experts; ++i)
                if (work[i] > best_val) {
                    best_val = work[i];
                    best_idx = i;
                }
            ids[t * top_k + k] = (int32_t)best_idx;
            weights[t * top_k + k] = best_val;
            work[best_idx] = -INFINITY;
        }
    }
    free(work);
}

/* topk_desc, src/gravity_glm.rs:230-240: descending, equal values keep
 * ascending index order.  Selection with an explicit taken mask gives the
 * same prefix as the stable sort, including -inf entries. */
void hko_topk_desc(const float* values, size_t n, size_t k, int32_t* out) {
    unsigned char* taken = (unsigned char*)calloc(n ? n : 1, 1);
    if (!taken) return;
    if (k > n) k = n;
    for (size_t r = 0; r < k; ++r) {
        size_t best = n;
        for (size_t i = 0; i < n; ++i) {
            if (taken[i]) continue;
            if (best == n || values[i] > values[best]) best = i;
        }
        taken[best] = 1;
        out[r] = (int32_t)best;
    }
    free(taken);
}

/* noaux_tc router, src/gravity_glm.rs:447-500. */
int hko_router_noaux_tc(const float* logits, const float* bias, size_t n_experts, size_t n_group,
                        size_t topk_group, size_t top_k, int norm_topk_prob,
                        float routed_scaling_factor, int32_t* ids, float* weights) {
    if (n_group == 0 || n_experts % n_group || topk_group == 0 || topk_group > n_group ||
        top_k == 0 || top_k > n_experts)
        return HKO_E_INVALID_ARG;
    size_t per_group = n_experts / n_group;
    if (top_k > topk_group * per_group) return HKO_E_INVALID_ARG;
    float* scores = (float*)malloc(n_experts * sizeof(float));
    float* corrected = (float*)malloc(n_experts * sizeof(float));
    float* choice = (float*)malloc(n_experts * sizeof(float));
    float* gscores = (float*)malloc(n_group * sizeof(float));
    int32_t* tmp = (int32_t*)malloc((n_experts + 2) * sizeof(int32_t));
    if (!scores || !corrected || !choice || !gscores || !tmp) {
        free(scores); free(corrected); free(choice); free(gscores); free(tmp);
        return HKO_E_INVALID_ARG;
    }
    for (size_t i = 0; i < n_experts; ++i) {
        scores[i] = 1.0f / (1.0f + expf(-logits[i]));
        corrected[i] = scores[i] + bias[i];
    }
    size_t two = per_group < 2 ? per_group : 2;
    for (size_t g = 0; g < n_group; ++g) {
        const float* slice = corrected + g * per_group;
        hko_topk_desc(slice, per_group, two, tmp);
        float s = -0.0f;
        for (size_t j = 0; j < two; ++j) s += slice[tmp[j]];
        gscores[g] = s;
    }
    int32_t* chosen = tmp;
    hko_topk_desc(gscores, n_group, topk_group, chosen);
    for (size_t i = 0; i < n_experts; ++i) choice[i] = -INFINITY;
    for (size_t c = 0; c < topk_group; ++c) {
        size_t g = (size_t)chosen[c];
        for (size_t e = g * per_group; e < (g + 1) * per_group; ++e) choice[e] = corrected[e];
    }
    hko_topk_desc(choice, n_experts, top_k, ids);
    for (size_t r = 0; r < top_k; ++r) weights[r] = scores[ids[r]];
    if (norm_topk_prob) {
        float total = -0.0f;
        for (size_t r = 0; r < top_k; ++r) total += weights[r];
        total = total + 1e-20f;
        for (size_t r = 0; r < top_k; ++r) weights[r] /= total;
    }
    for (size_t r = 0; r < top_k; ++r) weights[r] *= routed_scaling_factor;
    free(scores); free(corrected); free(choice); free(gscores); free(tmp);
    return HKO_OK;
}

/* source_qwen80_residual_rms_norm, qwen80_complete_runtime.rs:6778-6797. */
int hko_rmsnorm_1p(const float* x, const float* w, size_t n, float eps, float* out) {
    if (n == 0) return HKO_E_GEOMETRY;
    float sq = -0.0f;
    for (size_t i = 0; i < n; ++i) sq += x[i] * x[i];
    float variance = sq / (float)n;
    float inverse_rms = 1.0f / sqrtf(variance + eps);
    for (size_t i = 0; i < n; ++i) {
        out[i] = x[i] * inverse_rms * (1.0f + w[i]);
        if (!isfinite(out[i])) return HKO_E_NONFINITE;
    }
    return HKO_OK;
}

/* The greedy pick of terminal_greedy (qwen80_mixed_hybrid_decode.rs:3775-3788):
 * logits at n_valid.. are masked; best starts at (index 0, -inf) and moves on
 * v > best (NaN never wins, ties keep the lower index); a best that is not
 * finite (all masked, -inf or NaN, or a +inf winner) is an error. */
int hko_argmax_greedy(const float* logits, size_t n_valid, int32_t* token) {
    size_t best_i = 0;
    float best_v = -INFINITY;
    for (size_t i = 0; i < n_valid; ++i) {
        float v = logits[i];
        if (v > best_v || (v == best_v && i < best_i)) {
            best_v = v;
            best_i = i;
        }
    }
    *token = (int32_t)best_i;
    return isfinite(best_v) ? HKO_OK : HKO_E_NONFINITE;
}

/* terminal_greedy (qwen80_mixed_hybrid_decode.rs:3754-3790): residual
 * RMSNorm(1+w) of the final hidden state, the lm_head matvec (an HGRAVU01
 * uniform q8 G64 organ, uniform_factor_matvec_f32), then the greedy pick over
 * the first n_valid logits.  logits (vocab floats) receives the matvec. */
int hko_terminal_greedy(const float* hidden, const float* norm_w, size_t hidden_n, float eps, const uint16_t* scales,
                        const uint8_t* codes, size_t vocab, size_t n_valid, float* logits, int32_t* token) {
    if (n_valid == 0 || n_valid > vocab) return HKO_E_GEOMETRY;
    float* xn = (float*)malloc(hidden_n * sizeof(float));
    if (!xn) return HKO_E_INVALID_ARG;
    int rc = hko_rmsnorm_1p(hidden, norm_w, hidden_n, eps, xn);
    if (rc == HKO_OK) rc = hko_uniform_matvec(scales, codes, vocab, hidden_n, 8, 64, xn, logits);
    free(xn);
    if (rc) return rc;
    return hko_argmax_greedy(logits, n_valid, token);
}

/* silu_mul, src/kernels/mod.rs:24-31. */
void hko_silu_mul(const float* gate, const float* up, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        out[i] = s * up[i];
    }
}

/* ------------------------------------------------------------------------ */
/* Organs, MLP, MoE layer                                                    */
/* ------------------------------------------------------------------------ */

/* MixedPackedTensor::cpu_matvec (q80_mixed_decode.rs:1362-1369) for the
 * mixed-1p5 kinds, and the Q4/binary/mixed organs. */
int hko_organ_matvec(const hko_organ* o, const float* x, float* y) {
    switch (o->kind) {
    case 0: return hko_q4_matvec(o->scales, o->codes, o->rows, o->cols, o->group, x, y);
    case 1: return hko_bin_matvec(o->scales, o->codes, o->rows, o->cols, o->group, x, y);
    case 2: return hko_mixed_matvec(o->mixed, x, y);
    case 3: return hko_uniform_matvec(o->scales, o->codes, o->rows, o->cols, 8, 64, x, y);
    case 4: return hko_hgravs01_matvec(o->scales, o->codes, o->rows, o->rank, o->r_scales, o->r_codes, o->cols, 3, 64,
                                       x, y);
    case 5: return hko_rice_q1_matvec(o->scales, o->codes, o->rows, o->cols, o->res_indices, o->res_signs,
                                      o->res_count, o->res_scale, x, y);
    default: return HKO_E_UNSUPPORTED;
    }
}

int hko_organ_matvec_f64(const hko_organ* o, const double* x, double* y) {
    switch (o->kind) {
    case 0: return hko_q4_matvec_f64(o->scales, o->codes, o->rows, o->cols, o->group, x, y);
    case 1: return hko_bin_matvec_f64(o->scales, o->codes, o->rows, o->cols, o->group, x, y);
    case 2: return hko_mixed_matvec_f64(o->mixed, x, y);
    case 3: return hko_uniform_matvec_f64(o->scales, o->codes, o->rows, o->cols, 8, 64, x, y);
    case 4: {
        double* mid = (double*)malloc(o->rank * sizeof(double));
        if (!mid) return HKO_E_INVALID_ARG;
        int rc = hko_uniform_matvec_f64(o->r_scales, o->r_codes, o->rank, o->cols, 3, 64, x, mid);
        if (rc == HKO_OK) rc = hko_uniform_matvec_f64(o->scales, o->codes, o->rows, o->rank, 3, 64, mid, y);
        free(mid);
        return rc;
    }
    case 5: return hko_rice_q1_matvec_f64(o->scales, o->codes, o->rows, o->cols, o->res_indices, o->res_signs,
                                          o->res_count, o->res_scale, x, y);
    default: return HKO_E_UNSUPPORTED;
    }
}

/* source_qwen80_mlp, qwen80_complete_runtime.rs:6074-6107. */
int hko_mlp(const hko_organ* gate, const hko_organ* up, const hko_organ* down, const float* x,
            float* act, float* out) {
    size_t inter = gate->rows;
    if (up->rows != inter || down->cols != inter || gate->cols != up->cols) return HKO_E_GEOMETRY;
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = act ? act : (float*)malloc(inter * sizeof(float));
    int rc = HKO_E_INVALID_ARG;
    if (!g || !u || !a) goto done;
    if ((rc = hko_organ_matvec(gate, x, g)) != HKO_OK) goto done;
    if ((rc = hko_organ_matvec(up, x, u)) != HKO_OK) goto done;
    for (size_t i = 0; i < inter; ++i) {
        a[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        if (!isfinite(a[i])) {
            rc = HKO_E_NONFINITE;
            goto done;
        }
    }
    rc = hko_organ_matvec(down, a, out);
done:
    free(g);
    free(u);
    if (!act) free(a);
    return rc;
}

/* moe_suffix, qwen80_uniform_q4_hybrid_decode.rs:2615-2757. */
int hko_moe_layer_forward(const hko_moe_layer* L, const float* h, float* out, int32_t* ids_out,
                          float* weights_out, float* xn_out, float* logits_out) {
    size_t H = L->hidden, E = L->n_experts, K = L->top_k;
    int rc = HKO_E_INVALID_ARG;
    float* xn = (float*)malloc(H * sizeof(float));
    float* shared = (float*)calloc(H, sizeof(float));
    float* logits = (float*)malloc(E * sizeof(float));
    float* combined = (float*)calloc(H, sizeof(float));
    float* eout = (float*)malloc(H * sizeof(float));
    int32_t* ids = (int32_t*)malloc(K * sizeof(int32_t));
    float* wts = (float*)malloc(K * sizeof(float));
    if (!xn || !shared || !logits || !combined || !eout || !ids || !wts) goto done;
    if ((rc = hko_rmsnorm_1p(h, L->norm_w, H, L->eps, xn)) != HKO_OK) goto done;
    if (L->shared && (rc = hko_mlp(&L->shared[0], &L->shared[1], &L->shared[2], xn, NULL, shared)) != HKO_OK)
        goto done;
    hko_gemv_f32(L->router_w, E, H, xn, logits);
    if ((rc = hko_router_softmax_topk(logits, E, K, L->tie_eps, ids, wts)) != HKO_OK) goto done;
    for (size_t r = 0; r < K; ++r) {
        const hko_organ* ex = L->experts + (size_t)ids[r] * 3;
        if ((rc = hko_mlp(&ex[0], &ex[1], &ex[2], xn, NULL, eout)) != HKO_OK) goto done;
        for (size_t i = 0; i < H; ++i) combined[i] += eout[i] * wts[r];
    }
    if (L->shared) {
        float gate_val = 1.0f;
        if (L->shared_gate_w) {
            float logit = 0.0f;
            for (size_t i = 0; i < H; ++i) logit += L->shared_gate_w[i] * xn[i];
            gate_val = 1.0f / (1.0f + expf(-logit));
            if (!isfinite(gate_val) || gate_val < 0.0f || gate_val > 1.0f) {
                rc = HKO_E_NONFINITE;
                goto done;
            }
        }
        for (size_t i = 0; i < H; ++i) combined[i] += shared[i] * gate_val;
    }
    for (size_t i = 0; i < H; ++i) {
        out[i] = h[i] + combined[i];
        if (!isfinite(out[i])) {
            rc = HKO_E_NONFINITE;
            goto done;
        }
    }
    if (ids_out) memcpy(ids_out, ids, K * sizeof(int32_t));
    if (weights_out) memcpy(weights_out, wts, K * sizeof(float));
    if (xn_out) memcpy(xn_out, xn, H * sizeof(float));
    if (logits_out) memcpy(logits_out, logits, E * sizeof(float));
    rc = HKO_OK;
done:
    free(xn); free(shared); free(logits); free(combined); free(eout); free(ids); free(wts);
    return rc;
}

static int mlp_f64(const hko_organ* o, const double* x, double* out) {
    size_t inter = o[0].rows;
    double* g = (double*)malloc(inter * sizeof(double));
    double* u = (double*)malloc(inter * sizeof(double));
    int rc = HKO_E_INVALID_ARG;
    if (!g || !u) goto done;
    if ((rc = hko_organ_matvec_f64(&o[0], x, g)) != HKO_OK) goto done;
    if ((rc = hko_organ_matvec_f64(&o[1], x, u)) != HKO_OK) goto done;
    for (size_t i = 0; i < inter; ++i) g[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
    rc = hko_organ_matvec_f64(&o[2], g, out);
done:
    free(g);
    free(u);
    return rc;
}

/* FP64 authority (src/numeric_parity.rs:323-337 style): the same layer with
 * every intermediate in f64, routing fixed to the given ids; the routed
 * weights are the f64 softmax renormalised over those ids. */
int hko_moe_layer_forward_f64(const hko_moe_layer* L, const double* h, const int32_t* ids,
                              const float* weights_unused, double* out) {
    (void)weights_unused;
    size_t H = L->hidden, E = L->n_experts, K = L->top_k;
    int rc = HKO_E_INVALID_ARG;
    double* xn = (double*)malloc(H * sizeof(double));
    double* shared = (double*)calloc(H, sizeof(double));
    double* logits = (double*)malloc(E * sizeof(double));
    double* combined = (double*)calloc(H, sizeof(double));
    double* eout = (double*)malloc(H * sizeof(double));
    if (!xn || !shared || !logits || !combined || !eout) goto done;
    double sq = 0.0;
    for (size_t i = 0; i < H; ++i) sq += h[i] * h[i];
    double inv = 1.0 / sqrt(sq / (double)H + (double)L->eps);
    for (size_t i = 0; i < H; ++i) xn[i] = h[i] * inv * (1.0 + (double)L->norm_w[i]);
    for (size_t e = 0; e < E; ++e) {
        double acc = 0.0;
        for (size_t i = 0; i < H; ++i) acc += (double)L->router_w[e * H + i] * xn[i];
        logits[e] = acc;
    }
    double mx = -INFINITY, den = 0.0, sel = 0.0;
    for (size_t e = 0; e < E; ++e) mx = logits[e] > mx ? logits[e] : mx;
    for (size_t e = 0; e < E; ++e) den += exp(logits[e] - mx);
    for (size_t r = 0; r < K; ++r) sel += exp(logits[ids[r]] - mx) / den;
    for (size_t r = 0; r < K; ++r) {
        double w = exp(logits[ids[r]] - mx) / den / sel;
        if ((rc = mlp_f64(L->experts + (size_t)ids[r] * 3, xn, eout)) != HKO_OK) goto done;
        for (size_t i = 0; i < H; ++i) combined[i] += eout[i] * w;
    }
    if (L->shared) {
        if ((rc = mlp_f64(L->shared, xn, shared)) != HKO_OK) goto done;
        double gv = 1.0;
        if (L->shared_gate_w) {
            double lg = 0.0;
            for (size_t i = 0; i < H; ++i) lg += (double)L->shared_gate_w[i] * xn[i];
            gv = 1.0 / (1.0 + exp(-lg));
        }
        for (size_t i = 0; i < H; ++i) combined[i] += shared[i] * gv;
    }
    for (size_t i = 0; i < H; ++i) out[i] = h[i] + combined[i];
    rc = HKO_OK;
done:
    free(xn); free(shared); free(logits); free(combined); free(eout);
    return rc;
}

/* routed_moe, src/gravity_glm.rs:550-600: the router (:447-500), the
 * per-expert dense_mlp of batched_mlp (:503-548, experts are independent, so
 * one at a time here), routed accumulated in ascending expert id
 * (`order.sort_by_key(|&s| indices[s])`, then `*r += o * w`), then the shared
 * expert added with weight 1. */
int hko_noaux_moe_forward(const hko_noaux_moe* M, const float* x, float* out, int32_t* ids_out,
                          float* weights_out, float* logits_out) {
    size_t H = M->hidden, E = M->n_experts, K = M->top_k;
    int rc = HKO_E_INVALID_ARG;
    float* logits = (float*)malloc(E * sizeof(float));
    float* eout = (float*)malloc(H * sizeof(float));
    float* shared = (float*)malloc(H * sizeof(float));
    int32_t* ids = (int32_t*)malloc(K * sizeof(int32_t));
    float* wts = (float*)malloc(K * sizeof(float));
    size_t* order = (size_t*)malloc(K * sizeof(size_t));
    if (!logits || !eout || !shared || !ids || !wts || !order) goto done;
    hko_gemv_f32(M->router_w, E, H, x, logits);
    rc = hko_router_noaux_tc(logits, M->bias, E, M->n_group, M->topk_group, K, M->norm_topk_prob,
                             M->routed_scaling_factor, ids, wts);
    if (rc != HKO_OK) goto done;
    /* stable sort of the slots by expert id (ids are distinct) */
    for (size_t s = 0; s < K; ++s) order[s] = s;
    for (size_t s = 1; s < K; ++s) {
        size_t v = order[s], j = s;
        while (j > 0 && ids[order[j - 1]] > ids[v]) {
            order[j] = order[j - 1];
            --j;
        }
        order[j] = v;
    }
    for (size_t i = 0; i < H; ++i) out[i] = 0.0f;
    for (size_t s = 0; s < K; ++s) {
        size_t slot = order[s];
        const hko_organ* ex = M->experts + (size_t)ids[slot] * 3;
        if ((rc = hko_mlp(&ex[0], &ex[1], &ex[2], x, NULL, eout)) != HKO_OK) goto done;
        for (size_t i = 0; i < H; ++i) out[i] += eout[i] * wts[slot];
    }
    if (M->shared) {
        if ((rc = hko_mlp(&M->shared[0], &M->shared[1], &M->shared[2], x, NULL, shared)) != HKO_OK) goto done;
        for (size_t i = 0; i < H; ++i) out[i] += shared[i];
    }
    for (size_t i = 0; i < H; ++i) {
        if (!isfinite(out[i])) {
            rc = HKO_E_NONFINITE;
            goto done;
        }
    }
    if (ids_out) memcpy(ids_out, ids, K * sizeof(int32_t));
    if (weights_out) memcpy(weights_out, wts, K * sizeof(float));
    if (logits_out) memcpy(logits_out, logits, E * sizeof(float));
    rc = HKO_OK;
done:
    free(logits); free(eout); free(shared); free(ids); free(wts); free(order);
    return rc;
}

int hko_noaux_moe_forward_f64(const hko_noaux_moe* M, const double* x, const int32_t* ids, double* out) {
    size_t H = M->hidden, E = M->n_experts, K = M->top_k;
    int rc = HKO_E_INVALID_ARG;
    double* eout = (double*)malloc(H * sizeof(double));
    double* w = (double*)malloc(K * sizeof(double));
    if (!eout || !w) goto done;
    double total = 0.0;
    for (size_t r = 0; r < K; ++r) {
        if (ids[r] < 0 || (size_t)ids[r] >= E) goto done;
        double acc = 0.0;
        for (size_t i = 0; i < H; ++i) acc += (double)M->router_w[(size_t)ids[r] * H + i] * x[i];
        w[r] = 1.0 / (1.0 + exp(-acc));
        total += w[r];
    }
    for (size_t r = 0; r < K; ++r) {
        if (M->norm_topk_prob) w[r] /= total + 1e-20;
        w[r] *= (double)M->routed_scaling_factor;
    }
    for (size_t i = 0; i < H; ++i) out[i] = 0.0;
    for (size_t r = 0; r < K; ++r) {
        if ((rc = mlp_f64(M->experts + (size_t)ids[r] * 3, x, eout)) != HKO_OK) goto done;
        for (size_t i = 0; i < H; ++i) out[i] += eout[i] * w[r];
    }
    if (M->shared) {
        if ((rc = mlp_f64(M->shared, x, eout)) != HKO_OK) goto done;
        for (size_t i = 0; i < H; ++i) out[i] += eout[i];
    }
    rc = HKO_OK;
done:
    free(eout);
    free(w);
    return rc;
}

/* relative_l2, src/numeric_parity.rs:323-337. */
double hko_relative_l2_f64ref(const float* candidate, const double* reference, size_t n) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double d = (double)candidate[i] - reference[i];
        num += d * d;
        den += reference[i] * reference[i];
    }
    if (den == 0.0) return num == 0.0 ? 0.0 : INFINITY;
    return sqrt(num) / sqrt(den);
}

double hko_relative_l2_f32(const float* candidate, const float* reference, size_t n) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double d = (double)candidate[i] - (double)reference[i];
        num += d * d;
        den += (double)reference[i] * (double)reference[i];
    }
    if (den == 0.0) return num == 0.0 ? 0.0 : INFINITY;
    return sqrt(num) / sqrt(den);
}
