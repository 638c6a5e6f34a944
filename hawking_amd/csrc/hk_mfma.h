// hk_mfma.h -- the int8 matrix-core GEMV engine for packed organs (device).
//
// Batch-1 GEMV is bandwidth bound, but decoding 1-bit or 4-bit weights to
// floats costs at least one VALU op per weight, more than the VALU can issue
// at HBM speed for binary weights (8 weights per byte).  So the decode is
// moved into v_mfma_i32_16x16x64_i8:
//
//   * x is converted once per workgroup to fixed-point integers, one exponent
//     per zero-point unit (the SXG columns a lane's product covers):
//     X = rint(x * 2^E_u) with E_u = 23 - exponent(max |x| over the unit)
//     (|X| <= 2^23), and X * 2^k is split into four signed base-256 "limbs".
//     A unit's sums are scaled back by f_u = 2^(E - E_u) (E the exponent of
//     the whole vector's max, f_u <= 1, exact), so every element keeps 24
//     bits relative to its own unit's max, as an f32 product would, even
//     when one element of x is orders of magnitude above the rest.  The MFMA
//     A operand (16 x 64) holds, in row m = 4*slot + limb, the limbs of the
//     columns that lane-group `slot` of the B operand covers (zero elsewhere),
//     so one MFMA yields exact int32 partial sums for 4 column groups x 4
//     limbs of 16 weight rows.
//   * The B operand (64 x 16) comes straight from the packed bytes with one AND
//     per 4 weights: a binary bit plane s is bytes & (0x01 << s) = bit * 2^s, a
//     Q4 nibble plane is bytes & 0x0F, a Q2 field is bytes & (0x03 << 2u); the
//     power of two is folded into the A limbs (X * 2^(7-s) etc.).  A 3-bit code
//     is split into its low 2-bit field and its high bit, each its own B bytes
//     (the high bit's A carries the extra factor 4).  Binary plane
//     7 is the raw signed byte (no AND): its A row is -X7 and every lower
//     plane's A row carries +X7, which cancels the lower bits the raw byte
//     brings in (sum_s<7 (X_s 2^(7-s) + X7) 2^s b_s - X7 byte = 128 sum X_s b_s).
//     A mixed Q2 item's top field is read in place (bytes & 0xC0, with bit 7
//     stored inverted: 64 (code - 2) as a signed byte), so no field needs a shift.
//   * Per (row, group) the four int32 limbs are combined (pairs exactly in
//     int32, then one f32 fma), scaled by the unit's alpha * f_u and the zero
//     point removed with its beta * f_u * (sum of X) (binary: sum (2b-1) X =
//     2 sum bX - sum X; Q4: sum (n-8) X; Q2: sum (c-1.5) X) -- the x image
//     stores both per unit, so this is one fma as with a single exponent --
//     and the f16 group scale is applied; y = 2^-E * sum over groups.
//   * A tiles live in LDS in compact form: per tile 16 lanes x 16 B of limbs
//     plus a 16-byte zero block (stride 272 B); a lane whose row slot differs
//     from its column slot reads the zero block through a per-lane constant
//     offset, so the operand fetch is one ds_read_b128 with no VALU work.  One
//     A fetch feeds R row tiles.
// Weights arrive in the tiled layout of hk_tile.h.  Numerics: the only
// roundings are X (2^-24 of its unit's max |x|), the f32 limb combine and the
// f32 accumulation over groups; rel-L2 vs the serial f32 reference is ~1e-7.
#pragma once

#include "hk_internal.h"
#include "hk_tile.h"

namespace hk {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(const v4i& a, const v4i& b, const v4i& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <int KIND>
struct Kcfg;
// P = A tiles per step, SXG = columns per unit (the zero-point granularity a
// lane needs per step: one binary group, one Q4 group of 32, one Q2 half-group;
// each unit has its own exponent), SXW = floats stored per unit: {ALPHA f_u,
// BETA f_u sum X} (mixed: {alpha, correction} of binary items, then of Q2
// items, all times f_u; a lane reads the pair of its item's kind).  A lane's
// partial for a unit is combine(c) * pair[0] - pair[1] (in units of 2^-E).
template <>
struct Kcfg<HK_BIN> {
    static constexpr int P = 8, STEP_COLS = 512, DATA = 16, SXG = 128, SXW = 2;
    static constexpr float ALPHA = 1.0f / 64.0f, BETA = 1.0f;  // 2 sum bX - sum X
};
template <>
struct Kcfg<HK_Q4> {
    static constexpr int P = 2, STEP_COLS = 128, DATA = 16, SXG = 32, SXW = 2;
    static constexpr float ALPHA = 1.0f, BETA = 8.0f;  // sum (n - 8) X
};
template <>
struct Kcfg<HK_MIXED> {
    static constexpr int P = 8, STEP_COLS = 512, DATA = 32, SXG = 64, SXW = 4;
    static constexpr float ALPHA = 2.0f / 64.0f, BETA = 1.0f;  // binary items (Q2 items: alpha / 2)
};
template <>
struct Kcfg<HK_Q8> {
    static constexpr int P = 1, STEP_COLS = 64, DATA = 16, SXG = 16, SXW = 2;
    static constexpr float ALPHA = 1.0f, BETA = -1.0f;  // code ^ 0x80 = code - 128: + sum X
};
template <>
struct Kcfg<HK_U3> {
    static constexpr int P = 4, STEP_COLS = 128, DATA = 12, SXG = 32, SXW = 2;
    static constexpr float ALPHA = 1.0f / 32.0f, BETA = 3.0f;  // 32 code X, code = q + 3
};

constexpr int A_TILE_STRIDE = 272;  // 256 B of active-lane limbs + 16 B of zeros

// Bytes of the x image of an organ with `steps` steps: the A tiles, then the
// per-unit (SXG columns) scale factors and sums of X (SXW floats each).
template <int KIND>
__host__ __device__ constexpr size_t x_lds_bytes(uint32_t steps) {
    return (size_t)steps * Kcfg<KIND>::P * A_TILE_STRIDE +
           (size_t)steps * (Kcfg<KIND>::STEP_COLS / Kcfg<KIND>::SXG) * Kcfg<KIND>::SXW * 4;
}
// Columns of the image: cols rounded up to whole steps.
template <int KIND>
__host__ __device__ constexpr uint32_t x_image_cols(uint32_t steps) {
    return steps * (uint32_t)Kcfg<KIND>::STEP_COLS;
}

// c[0] + 2^8 c[1] + 2^16 c[2] + 2^24 c[3].  Every limb sum is below 2^21 in
// magnitude (at most 128 products of a limb byte and a B byte, each <= 2^14),
// so each pair combines exactly in int32 before the one f32 rounding.
__device__ __forceinline__ float combine_limbs(const v4i& c) {
    const int lo = c[0] + c[1] * 256, hi = c[2] + c[3] * 256;
    return __builtin_fmaf((float)hi, 65536.0f, (float)lo);
}

// Value of A byte i (0..15) for step t, MFMA mu, column slot q, from the
// quantized x (X as exact integer-valued floats, zero past cols).
template <int KIND>
__device__ __forceinline__ int32_t a_value(const float* xq, int t, int mu, int q, int i) {
    auto X = [&](uint32_t c) { return (int32_t)xq[c]; };
    if constexpr (KIND == HK_BIN) {
        const uint32_t c0 = (uint32_t)(t * 512 + q * 128 + 8 * i);
        const int32_t v7 = X(c0 + 7u);
        if (mu == 7) return -v7;
        return X(c0 + (uint32_t)mu) * (1 << (7 - mu)) + v7;
    } else if constexpr (KIND == HK_Q4) {
        return X((uint32_t)(t * 128 + q * 32 + 2 * i + mu));
    } else if constexpr (KIND == HK_Q8) {
        return X((uint32_t)(t * 64 + q * 16 + i));
    } else if constexpr (KIND == HK_U3) {
        // MFMA mu: dwords 0-1 are the low fields u = mu of low dwords 0-1
        // (column 16d + 4j + mu, times 4^mu; mu = 3 is shifted down to 1),
        // dwords 2-3 the high bits s = 2mu, 2mu+1 (column 8j + s, times 2^s,
        // bit 7 as the signed byte -128); every product is scaled to 32 * code * X
        const int d = i >> 2, j = i & 3;
        const uint32_t c0 = (uint32_t)(t * 128 + q * 32);
        if (d < 2) return X(c0 + (uint32_t)(16 * d + 4 * j + mu)) * (mu == 3 ? 32 : 1 << (5 - 2 * mu));
        const int s = 2 * mu + d - 2;
        const int32_t v = X(c0 + (uint32_t)(8 * j + s));
        return s == 7 ? -v : v * (1 << (7 - s));
    } else {
        const int h = mu >> 2, u = mu & 3, r = i >> 2, j = i & 3;
        const int a = r < 2 ? 2 * h + r : 2 * h + 2 + r;
        const int32_t v = X((uint32_t)(t * 512 + q * 128) + mixed_q2_col((uint32_t)a, (uint32_t)j, (uint32_t)u));
        return v * (1 << (6 - 2 * u));
    }
}

// The threads that build one x image together: the whole block, or one wave
// building an image of its own (no block barrier).
struct BlockTeam {
    __device__ uint32_t idx() const { return threadIdx.x; }
    __device__ uint32_t size() const { return blockDim.x; }
    __device__ float reduce_max(float m, float* red) const {
        m = wave_max(m);
        const int nw = (int)(blockDim.x >> 6);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        __syncthreads();
        float r = red[0];
        for (int w = 1; w < nw; ++w) r = fmaxf(r, red[w]);
        return r;
    }
    __device__ void sync() const { __syncthreads(); }
};
struct WaveTeam {
    uint32_t lane;
    __device__ uint32_t idx() const { return lane; }
    __device__ uint32_t size() const { return 64u; }
    __device__ float reduce_max(float m, float*) const { return wave_max(m); }
    __device__ void sync() const {}
};

// x is consumed in chunks of 8 consecutive columns: team member m owns chunks
// m, m + size, m + 2 size, ...  The first NC of them are loaded into
// registers by load_x, which a kernel issues before its weight prefetch so
// that waiting for x does not wait for the weights; later chunks are read
// from x again when needed.  Requires cols % 8 == 0 and a 16-byte aligned x.
template <int NC>
struct XChunks {
    float4 v[NC][2];
};

// The load is unconditional (a chunk past cols re-reads the last one and is
// zeroed after): a load under a per-lane condition would wait for the one
// before it.
__device__ __forceinline__ void load_chunk(const float* x, uint32_t c0, uint32_t cols, float4* v) {
    const uint32_t c = min(c0, cols - 8u);
    v[0] = *reinterpret_cast<const float4*>(x + c);
    v[1] = *reinterpret_cast<const float4*>(x + c + 4);
    if (c0 >= cols) v[0] = v[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

template <int NC, class Team>
__device__ __forceinline__ void load_x(const Team& team, const float* x, uint32_t cols, XChunks<NC>& xc) {
#pragma unroll
    for (int j = 0; j < NC; ++j) load_chunk(x, 8u * (team.idx() + (uint32_t)j * team.size()), cols, xc.v[j]);
}

// max |v| of a chunk, +inf if any element is NaN (fmaxf drops NaN operands,
// so a NaN must become a value the max keeps for the non-finite check).
__device__ __forceinline__ float max_abs8(const float4* v) {
    const float m = fmaxf(fmaxf(fmaxf(fabsf(v[0].x), fabsf(v[0].y)), fmaxf(fabsf(v[0].z), fabsf(v[0].w))),
                          fmaxf(fmaxf(fabsf(v[1].x), fabsf(v[1].y)), fmaxf(fabsf(v[1].z), fabsf(v[1].w))));
    const float s = v[0].x + v[0].y + v[0].z + v[0].w + v[1].x + v[1].y + v[1].z + v[1].w;
    return s != s ? INFINITY : m;  // a NaN sum: a NaN, or +inf with -inf
}

__device__ __forceinline__ int32_t quantize8(const float4* v, int E, float* f) {
    const float in[8] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w};
    int32_t s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        f[k] = rintf(ldexpf(in[k], E));
        s += (int32_t)f[k];
    }
    return s;
}

// Reductions over aligned groups of G lanes (G a power of two <= 64) as an
// xor butterfly, every lane of a group getting its group's result: distances
// 1 and 2 are DPP quad permutations, 4 and 8 two DPP row shifts each (row_shl
// on the lower bank of every pair, row_shr on the upper, selected by the
// bank mask), 16 and 32 the permlane16 / permlane32 swaps.  No LDS round
// trip, unlike a shuffle; exact for integer sums and for max.  The lanes of a
// group must be active together.
template <int K>
__device__ __forceinline__ uint32_t xor_partner(uint32_t v) {
    const int x = (int)v;
    if constexpr (K == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
    if constexpr (K == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
    if constexpr (K == 4)  // row_shr:4 into banks 1, 3; row_shl:4 into banks 0, 2
        return (uint32_t)__builtin_amdgcn_update_dpp(__builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xA, false), x,
                                                     0x104, 0xF, 0x5, false);
    if constexpr (K == 8)  // row_shr:8 into banks 2, 3; row_shl:8 into banks 0, 1
        return (uint32_t)__builtin_amdgcn_update_dpp(__builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xC, false), x,
                                                     0x108, 0xF, 0x3, false);
}
template <int G, class Op>
__device__ __forceinline__ uint32_t group_reduce(uint32_t v, Op op) {
    if constexpr (G > 1) v = op(v, xor_partner<1>(v));
    if constexpr (G > 2) v = op(v, xor_partner<2>(v));
    if constexpr (G > 4) v = op(v, xor_partner<4>(v));
    if constexpr (G > 8) v = op(v, xor_partner<8>(v));
    if constexpr (G > 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = op(a[0], a[1]);
    }
    if constexpr (G > 32) {
        const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = op(b[0], b[1]);
    }
    return v;
}
template <int G>
__device__ __forceinline__ int32_t group_sum(int32_t v) {
    return (int32_t)group_reduce<G>((uint32_t)v, [](uint32_t a, uint32_t b) { return a + b; });
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
    return __uint_as_float(group_reduce<G>(__float_as_uint(v), [](uint32_t a, uint32_t b) {
        return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    }));
}

// A unit's exponent E_u is capped at UNIT_EXP_CAP above the image's: the
// unit entries fold f_u = 2^-E_u into ALPHA (down to 2^-6 for a Q2 item's
// half alpha), and 2^-6 * 2^-120 = 2^-126 is the smallest normal float.  A
// unit whose max is below 2^-98 therefore keeps fewer than 24 bits: its
// elements are quantized to 2^-120 (2^-121 worst-case error) instead.
constexpr int UNIT_EXP_CAP = 120;

// The x image: fixed-point x (E = 23 - exponent of max|x|; 0 for x = 0 or
// non-finite x, which sets the flag), per unit of SXG columns E_u = 23 -
// exponent of the unit's max (at most E + UNIT_EXP_CAP; E for an all-zero unit),
// X = rint(x 2^E_u), and from it the A tiles and each unit's {ALPHA f_u,
// BETA f_u sum X} with f_u = 2^(E - E_u), written to img
// (x_lds_bytes<KIND>(steps) bytes, any address space).  Returns E.
//
// The image columns (cols rounded up to whole steps, zero past cols) go in
// rounds of 8 * team size columns: each member quantizes its chunk of the
// round into the LDS window xq + j * xq_stride (exact integer-valued floats),
// then the team builds the round's steps from the window.  xq_stride = 0
// reuses one window of min(image columns, 8 * team size) floats; with
// xq_stride = 8 * team size and xq == x (x staged in LDS with room for the
// image columns) x is quantized in place, every chunk being read and
// rewritten by its owner only.  8 * team size must be a multiple of the
// step's columns.  Ends with team.sync().
//
// [tb, te) limits the build to those steps (E still comes from all of x), so
// several teams can build parts of one image; xq then stands for image column
// tb * step columns, and the register chunks are used only when tb = 0.
template <int KIND, int NC, class Team>
__device__ int x_image(const Team& team, const XChunks<NC>& xc, const float* x, uint32_t cols, uint32_t steps,
                       uint8_t* img, float* xq, uint32_t xq_stride, float* red, bool* nonfinite, uint32_t tb = 0,
                       uint32_t te = 0xFFFFFFFFu) {
    constexpr int P = Kcfg<KIND>::P, SC = Kcfg<KIND>::STEP_COLS, NL = Kcfg<KIND>::SXG / 8;
    const uint32_t me = team.idx(), ts = team.size();
    const uint32_t nch = steps * (uint32_t)SC / 8u, wcols = 8u * ts, rounds = (nch + ts - 1u) / ts;
    te = min(te, steps);
    const uint32_t cb = tb * (uint32_t)SC / 8u, ce = te * (uint32_t)SC / 8u;
    const uint32_t prounds = ce > cb ? (ce - cb + ts - 1u) / ts : 0u;
    float* SX = reinterpret_cast<float*>(img + (size_t)steps * P * A_TILE_STRIDE);
    uint32_t* A = reinterpret_cast<uint32_t*>(img);

    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; ++j) m = fmaxf(m, max_abs8(xc.v[j]));
    for (uint32_t j = NC; j < rounds; ++j) {
        float4 v[2];
        load_chunk(x, 8u * (me + j * ts), cols, v);
        m = fmaxf(m, max_abs8(v));
    }
    m = team.reduce_max(m, red);
    const bool bad = !isfinite(m);
    *nonfinite = bad;
    int e2 = 0;
    if (!bad && m > 0.0f) (void)frexpf(m, &e2);
    const int E = (!bad && m > 0.0f) ? 23 - e2 : 0;

    for (int i = (int)(tb * P * 4 + me); i < (int)te * P * 4; i += (int)ts)
        A[(i >> 2) * (A_TILE_STRIDE / 4) + 64 + (i & 3)] = 0u;

    auto round = [&](uint32_t j, float4* v) {
        float* w = xq + j * xq_stride;
        const uint32_t ch = cb + me + j * ts;
        if (ch < ce) {
            if (bad) v[0] = v[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            // a unit's NL chunks belong to NL consecutive members, all active together
            const float mu = group_max<NL>(max_abs8(v));
            int eu = 0;
            if (mu > 0.0f) (void)frexpf(mu, &eu);
            const int Eu = mu > 0.0f ? min(23 - eu, E + UNIT_EXP_CAP) : E;
            const float fu = ldexpf(1.0f, E - Eu);
            float f[8];
            int32_t s = quantize8(v, Eu, f);
            float4* o = reinterpret_cast<float4*>(w + 8u * me);
            o[0] = make_float4(f[0], f[1], f[2], f[3]);
            o[1] = make_float4(f[4], f[5], f[6], f[7]);
            s = group_sum<NL>(s);
            if constexpr (KIND == HK_MIXED) {
                // the Q2 top field (columns 6, 7 of every chunk) decodes as
                // code - 2, so its items subtract 1.5 sum X - 2 sum_top X
                // (3 sum X - 4 sum_top X < 2^31: exact in int32, halved exactly)
                const int32_t s3 = group_sum<NL>((int32_t)f[6] + (int32_t)f[7]);
                if ((me & (uint32_t)(NL - 1)) == 0)
                    reinterpret_cast<float4*>(SX)[ch / (uint32_t)NL] =
                        make_float4(Kcfg<KIND>::ALPHA * fu, (float)s * fu, 0.5f * Kcfg<KIND>::ALPHA * fu,
                                    (float)(3 * s - 4 * s3) * 0.5f * fu);
            } else {
                if ((me & (uint32_t)(NL - 1)) == 0)
                    reinterpret_cast<float2*>(SX)[ch / (uint32_t)NL] =
                        make_float2(Kcfg<KIND>::ALPHA * fu, Kcfg<KIND>::BETA * (float)s * fu);
            }
        }
        team.sync();
        // this round's steps; unit = (tau, slot q, dword d): 4 A bytes -> 4
        // lanes' dwords via a byte transpose
        const uint32_t t0 = tb + j * (wcols / (uint32_t)SC), t1 = min(t0 + wcols / (uint32_t)SC, te);
        const int nunits = (int)(t1 - t0) * P * 16;
        for (int u = (int)me; u < nunits; u += (int)ts) {
            const int d = u & 3, q = (u >> 2) & 3, tl = u >> 4;
            const int t = tl / P, mu = tl % P;
            uint32_t z[4];
#pragma unroll
            for (int jb = 0; jb < 4; ++jb)
                z[jb] = ((uint32_t)a_value<KIND>(w, t, mu, q, 4 * d + jb) + 0x80808080u) ^ 0x80808080u;
            const uint32_t tau = t0 * (uint32_t)P + (uint32_t)tl;
#pragma unroll
            for (int L = 0; L < 4; ++L) {
                // v_perm: selector 0..3 = byte of the second operand, 4..7 = byte of the first, 0x0c = 0
                const uint32_t lo = __builtin_amdgcn_perm(z[1], z[0], 0x0c0c0400u | (uint32_t)L | ((uint32_t)L << 8));
                const uint32_t hi = __builtin_amdgcn_perm(z[3], z[2], 0x04000c0cu | ((uint32_t)L << 16) | ((uint32_t)L << 24));
                A[tau * (A_TILE_STRIDE / 4) + (4 * q + L) * 4 + d] = lo | hi;
            }
        }
        team.sync();
    };
    const uint32_t jr = tb == 0 ? (uint32_t)NC : 0u;  // rounds served from the register chunks
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        if ((uint32_t)j >= min(jr, prounds)) break;
        float4 v[2] = {xc.v[j][0], xc.v[j][1]};
        round((uint32_t)j, v);
    }
    for (uint32_t j = min(jr, prounds); j < prounds; ++j) {
        float4 v[2];
        load_chunk(x, 8u * (cb + me + j * ts), cols, v);
        round(j, v);
    }
    return E;
}

// Where column c's A bytes go in an x image (a_value inverted): tile tau and
// the byte offset of limb 0 inside it (limb L at + 16 L), and the power of
// two the column's X is scaled by.
template <int KIND>
__device__ __forceinline__ void a_pos(uint32_t c, uint32_t& tau, uint32_t& off, int& sh) {
    static_assert(KIND == HK_MIXED || KIND == HK_Q4 || KIND == HK_Q8, "per-column scatter kinds");
    if constexpr (KIND == HK_MIXED) {
        // column i of the 128-column group q -> (a, j, u): tile mu = 4h + u,
        // byte 4r + j of rows 4q + limb
        const uint32_t i = c & 127u, h = i >> 6;
        const uint32_t av = ((i >> 5) & 3u) | ((i & 1u) << 2), j = (i >> 3) & 3u, u = (i >> 1) & 3u;
        const uint32_t r = (av & 3u) - 2u * h + ((i & 1u) ? 2u : 0u);
        tau = (c >> 9) * (uint32_t)Kcfg<KIND>::P + 4u * h + u;
        off = 64u * ((c >> 7) & 3u) + 4u * r + j;
        sh = 6 - 2 * (int)u;
    } else if constexpr (KIND == HK_Q4) {
        const uint32_t cs = c & 127u;
        tau = (c >> 7) * (uint32_t)Kcfg<KIND>::P + (cs & 1u);
        off = 64u * (cs >> 5) + ((cs & 31u) >> 1);
        sh = 0;
    } else {
        // q8: step = one tile of 64 columns, lane group (c / 16) % 4, byte c % 16
        tau = c >> 6;
        off = 64u * ((c >> 4) & 3u) + (c & 15u);
        sh = 0;
    }
}

// One chunk (8 columns, values v, zero past the organ's columns) of an x
// image with E = 0 (image_wave's unit rule), written at its tile positions
// relative to tile tau0 and to the unit entries of chunk cb on.  Every lane
// of the chunk's unit (SXG / 8 consecutive lanes) calls it together.
// Returns whether the unit held a non-finite value (then zeroed).
template <int KIND>
__device__ __forceinline__ bool image_chunk(uint32_t ch, float4 (&v)[2], uint8_t* tiles, float* sx, uint32_t cb,
                                            uint32_t tau0) {
    constexpr int NL = Kcfg<KIND>::SXG / 8;
    float m = group_max<NL>(max_abs8(v));
    const bool bad = !isfinite(m);
    if (bad) {
        v[0] = v[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        m = 0.0f;
    }
    int eu = 0;
    if (m > 0.0f) (void)frexpf(m, &eu);
    const int Eu = m > 0.0f ? min(23 - eu, UNIT_EXP_CAP) : 0;
    const float fu = ldexpf(1.0f, -Eu);
    float f[8];
    const int32_t s = group_sum<NL>(quantize8(v, Eu, f));
    if constexpr (KIND == HK_MIXED) {
        const int32_t s3 = group_sum<NL>((int32_t)f[6] + (int32_t)f[7]);
        if ((ch & (uint32_t)(NL - 1)) == 0)
            reinterpret_cast<float4*>(sx)[(ch - cb) / (uint32_t)NL] =
                make_float4(Kcfg<KIND>::ALPHA * fu, (float)s * fu, 0.5f * Kcfg<KIND>::ALPHA * fu,
                            (float)(3 * s - 4 * s3) * 0.5f * fu);
    } else {
        if ((ch & (uint32_t)(NL - 1)) == 0)
            reinterpret_cast<float2*>(sx)[(ch - cb) / (uint32_t)NL] =
                make_float2(Kcfg<KIND>::ALPHA * fu, Kcfg<KIND>::BETA * (float)s * fu);
    }
    if constexpr (KIND == HK_U3) {
        // a 3-bit step is 128 columns in 4 lane groups of 32; column o of a
        // group sits twice: as a low 2-bit field (tile o % 4, byte
        // 4 (o / 16) + (o / 4) % 4, times 4^(2 - o % 4), field 3 times 32)
        // and as a high bit s = o % 8 (tile s / 2, byte 4 (2 + s % 2) + o / 8,
        // times 2^(7 - s), bit 7 as -X): a_value's 3-bit rule inverted
        const uint32_t m = ch & 3u, base = 64u * ((ch >> 2) & 3u), tb = (ch >> 4) * 4u - tau0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int32_t x = (int32_t)f[e];
            const uint32_t mu = (uint32_t)e & 3u;
            const int32_t lo = x * (mu == 3u ? 32 : 1 << (5 - 2 * (int)mu));
            const int32_t hi = e == 7 ? -x : x * (1 << (7 - e));
            const uint32_t ilo = 4u * (m >> 1) + ((2u * m + ((uint32_t)e >> 2)) & 3u);
            const uint32_t ihi = 4u * (2u + ((uint32_t)e & 1u)) + m;
            const uint32_t zl = ((uint32_t)lo + 0x80808080u) ^ 0x80808080u;
            const uint32_t zh = ((uint32_t)hi + 0x80808080u) ^ 0x80808080u;
            uint8_t* pl = tiles + (size_t)(tb + mu) * A_TILE_STRIDE + base + ilo;
            uint8_t* ph = tiles + (size_t)(tb + ((uint32_t)e >> 1)) * A_TILE_STRIDE + base + ihi;
            pl[0] = (uint8_t)zl;
            pl[16] = (uint8_t)(zl >> 8);
            pl[32] = (uint8_t)(zl >> 16);
            pl[48] = (uint8_t)(zl >> 24);
            ph[0] = (uint8_t)zh;
            ph[16] = (uint8_t)(zh >> 8);
            ph[32] = (uint8_t)(zh >> 16);
            ph[48] = (uint8_t)(zh >> 24);
        }
    } else if constexpr (KIND == HK_BIN) {
        // the chunk is byte ch % 16 of lane group (ch / 16) % 4 in all 8 bit
        // planes of step ch / 64: plane mu < 7 holds X_mu 2^(7-mu) + X_7,
        // plane 7 holds -X_7 (a_value's binary rule)
        const uint32_t off = 64u * ((ch >> 4) & 3u) + (ch & 15u), tb = (ch >> 6) * 8u - tau0;
        const int32_t x7 = (int32_t)f[7];
#pragma unroll
        for (int mu = 0; mu < 8; ++mu) {
            const int32_t a = mu < 7 ? (int32_t)f[mu] * (1 << (7 - mu)) + x7 : -x7;
            const uint32_t z = ((uint32_t)a + 0x80808080u) ^ 0x80808080u;
            uint8_t* p = tiles + (size_t)(tb + (uint32_t)mu) * A_TILE_STRIDE + off;
            p[0] = (uint8_t)z;
            p[16] = (uint8_t)(z >> 8);
            p[32] = (uint8_t)(z >> 16);
            p[48] = (uint8_t)(z >> 24);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t tau, off;
            int sh;
            a_pos<KIND>(8u * ch + (uint32_t)e, tau, off, sh);
            // signed base-256 limbs of the scaled value
            const uint32_t z = ((uint32_t)((int32_t)f[e] * (1 << sh)) + 0x80808080u) ^ 0x80808080u;
            uint8_t* p = tiles + (size_t)(tau - tau0) * A_TILE_STRIDE + off;
            p[0] = (uint8_t)z;
            p[16] = (uint8_t)(z >> 8);
            p[32] = (uint8_t)(z >> 16);
            p[48] = (uint8_t)(z >> 24);
        }
    }
    return bad;
}

// The zero blocks (bytes 256..271) of the A tiles of `steps` steps.
template <int KIND>
__device__ __forceinline__ void image_zero_blocks(uint32_t lane, uint8_t* tiles, uint32_t steps) {
    for (uint32_t i = lane; i < steps * (uint32_t)Kcfg<KIND>::P; i += 64u)
        *reinterpret_cast<uint4*>(tiles + (size_t)i * A_TILE_STRIDE + 256u) = make_uint4(0u, 0u, 0u, 0u);
}

// The x image of x (cols columns, cols a multiple of 8; the image columns
// past cols are zero) with E = 0, or the part of it in chunks [cb, ce) of 8
// columns (whole steps), built by one wave straight into `tiles` (the A tiles
// from the range's first step on) and `sx` (the unit entries from the
// range's first unit on), in LDS or global memory: lane l takes chunks cb + l,
// cb + l + 64, ...; each unit (SXG
// columns = NL consecutive lanes) has E_u = 23 - exponent of its max (at most
// UNIT_EXP_CAP, so ALPHA f_u is a normal float; 0 for an all-zero unit), and every
// column's limbs of X = rint(x 2^E_u) are stored as bytes at their tile
// positions (a_pos).  These are the bytes x_image makes, and its unit entries
// divided by its 2^E (every scale a power of two times the same roundings),
// so a dot product on this image is x_image's times 2^-E exactly: no
// whole-vector maximum, no gather pass.  A non-finite value zeroes its unit
// and sets *nonfinite.  Touches only the image range it builds (no barrier).
template <int KIND>
__device__ void image_wave(uint32_t lane, const float* x, uint32_t cols, uint8_t* tiles, float* sx, uint32_t cb,
                           uint32_t ce, bool* nonfinite) {
    constexpr int P = Kcfg<KIND>::P, SC = Kcfg<KIND>::STEP_COLS;
    const uint32_t tau0 = cb * 8u / SC * P;
    image_zero_blocks<KIND>(lane, tiles, (ce - cb) * 8u / SC);
    bool any_bad = false;
    // a unit's NL chunks are NL consecutive lanes, active together (ranges are whole steps)
    for (uint32_t ch = cb + lane; ch < ce; ch += 64u) {
        float4 v[2];
        load_chunk(x, 8u * ch, cols, v);
        any_bad |= image_chunk<KIND>(ch, v, tiles, sx, cb, tau0);
    }
    *nonfinite = any_bad;
}

// Per-lane byte offset of this lane's A operand inside a tile.
__device__ __forceinline__ uint32_t a_lane_offset(int lane) {
    return (((lane & 15) >> 2) == (lane >> 4)) ? (uint32_t)(lane & 15) * 16u : 256u;
}

__device__ __forceinline__ v4i lds_a(const uint8_t* lds, uint32_t tau, uint32_t off) {
    return *reinterpret_cast<const v4i*>(lds + tau * A_TILE_STRIDE + off);
}

// A-operand source: an x image (in LDS) and this lane's offset into each tile.
struct ImageA {
    const uint8_t* img;
    uint32_t aoff;
    __device__ __forceinline__ v4i operator()(uint32_t tau) const { return lds_a(img, tau, aoff); }
};

// One step of R row tiles, as fetched from memory: the weight bytes and scales
// each lane needs (row lane%16 of tile T[r], column slot lane/16).
template <int KIND, int R>
struct Frag;
// Scales stay raw f16 bits until the step is consumed: converting at fetch
// time would wait for the load there and collapse the prefetch pipeline.
template <int R>
struct Frag<HK_BIN, R> {
    uint4 v[R];
    uint16_t s[R];
};
template <int R>
struct Frag<HK_Q4, R> {
    uint4 v[R];
    uint16_t s[R];
};
template <int R>
struct Frag<HK_Q8, R> {
    uint4 v[R];
    uint16_t s[R];
};
template <int R>
struct Frag<HK_U3, R> {
    uint2 lo[R];
    uint32_t hi[R];
    uint16_t s[R];
};
// q2m: the step's Q2 lane mask, wave-uniform (scalar registers); a lane's
// kind is its bit, read with inverse ballot (no vector register per step).
template <int R>
struct Frag<HK_MIXED, R> {
    uint32_t V[R][8];
    uint16_t s0[R], s1[R];
    uint64_t q2m[R];
};

// Issue the loads of a mixed step with header h into slot r of f.
template <int R>
__device__ __forceinline__ void fetch_mixed(const OrganView& o, const uint4& h, int lane, Frag<HK_MIXED, R>& f, int r) {
    // the header is wave-uniform: keep it in scalar registers
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(h.x), mhi = __builtin_amdgcn_readfirstlane(h.y);
    const uint32_t doff = __builtin_amdgcn_readfirstlane(h.z), soff = __builtin_amdgcn_readfirstlane(h.w);
    const uint64_t mask = ((uint64_t)mhi << 32) | mlo;
    const uint32_t below = __builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u));
    const bool isq2 = __builtin_amdgcn_inverse_ballot_w64(mask);
    // uniform bases (scalar registers) plus 32-bit lane offsets: the loads
    // take the scalar-base form, no 64-bit address arithmetic per lane
    const uint8_t* db = o.data + doff;
    const uint32_t dl = 16u * ((uint32_t)lane + below);
    const uint4 va = ldg(reinterpret_cast<const uint4*>(db + dl));
    // binary lanes re-read their 16 bytes (an exec-masked load measured slower)
    const uint4 vb = ldg(reinterpret_cast<const uint4*>(db + (dl + (isq2 ? 16u : 0u))));
    f.V[r][0] = va.x;
    f.V[r][1] = va.y;
    f.V[r][2] = va.z;
    f.V[r][3] = va.w;
    f.V[r][4] = vb.x;
    f.V[r][5] = vb.y;
    f.V[r][6] = vb.z;
    f.V[r][7] = vb.w;
    // one aligned 4-byte load per lane: a Q2 lane's pair, or the word that
    // holds a binary lane's scale (the step's Q2 pairs come first); a small
    // load costs the memory pipeline as much as a 16-byte one, so two u16
    // loads cost twice
    const uint32_t nq2 = (uint32_t)__builtin_popcountll(mask), j = (uint32_t)lane - below;
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(o.scales + soff);
    const uint32_t w = ldg(sw + (isq2 ? below : nq2 + (j >> 1)));
    const uint16_t lo = (uint16_t)w, hi = (uint16_t)(w >> 16);
    f.s0[r] = (isq2 || !(j & 1u)) ? lo : hi;
    f.s1[r] = isq2 ? hi : f.s0[r];
    f.q2m[r] = mask;
}

// Issue the loads of step t of tile T of organ o into slot r of f (a mixed
// step first loads its header, and its data loads wait for it).
//
// NT: the weight data (not the scales) of binary, Q4 and q8 steps load with
// the non-temporal hint.  Measured on 512 x 2048 organ streams: Q4 and q8
// 0.74 -> 0.84 of 8 TB/s, binary (with the 2-tile, 5-deep shape) 0.76 ->
// 0.78; the hint on the 2-byte scale loads, on the mixed kind's loads (its
// binary lanes re-read their 16 bytes) or on the 3-bit kind's measured
// slower, and so did the terminal head's q8 launch (its kernel runs NT =
// false).  The default is off: the batch-1 MoE decode kernels, bound by
// their latency chains, ran 1-2 % faster with ordinary loads.
template <int KIND, int R, bool NT = false>
__device__ __forceinline__ void fetch_one(const OrganView& o, uint32_t T, uint32_t t, int lane, Frag<KIND, R>& f,
                                          int r) {
    // offsets in 32 bits (an organ's tiled sections are below 4 GiB, checked
    // when it is created): a 64-bit product per address costs scalar
    // instructions on every step
    if constexpr (KIND == HK_BIN || KIND == HK_Q4) {
        const uint32_t st = T * o.steps + t;
        const uint4* p = reinterpret_cast<const uint4*>(o.data + (st * 1024u + 16u * (uint32_t)lane));
        f.v[r] = NT ? ldg_nt(p) : ldg(p);
        f.s[r] = ldg(o.scales + (st * 64u + (uint32_t)lane));
    } else if constexpr (KIND == HK_Q8) {
        const uint32_t st = T * o.steps + t;
        const uint4* p = reinterpret_cast<const uint4*>(o.data + (st * 1024u + 16u * (uint32_t)lane));
        f.v[r] = NT ? ldg_nt(p) : ldg(p);
        f.s[r] = ldg(o.scales + (st * 16u + (uint32_t)(lane & 15)));
    } else if constexpr (KIND == HK_U3) {
        // the last step stores tail_q slots; lanes of absent slots re-read slot 0
        const bool tail = t + 1 == o.steps;
        const uint32_t nq = tail ? o.tail_q : 4u;
        const uint32_t l = (uint32_t)(lane >> 4) < nq ? (uint32_t)lane : (uint32_t)(lane & 15);
        // the lane's 12 bytes (low fields, then high bits): one 12-byte load
        const uint32_t* lw = reinterpret_cast<const uint32_t*>(o.data + (T * (uint32_t)u3_tile_data(o.steps, o.tail_q) +
                                                                         768u * t + 12u * l));
        f.lo[r] = make_uint2(ldg(lw), ldg(lw + 1));
        f.hi[r] = ldg(lw + 2);
        // (a 32-bit byte offset: the scalar-base form; measured neutral or
        // slightly slower for the other kinds' scale loads, so only here)
        f.s[r] = ldg_at(o.scales, 2u * (T * (uint32_t)u3_tile_scales(o.steps, o.tail_q) + 64u * t + l));
    } else {
        fetch_mixed<R>(o, ldg(o.hdr + (T * o.steps + t)), lane, f, r);
    }
}

// Issue the loads of step t for tiles T[0..R-1] (tiles r >= nvalid alias T[0]).
template <int KIND, int R, bool NT = false>
__device__ __forceinline__ void fetch_step(const OrganView& o, const uint32_t* T, int nvalid, uint32_t t, int lane,
                                           Frag<KIND, R>& f) {
#pragma unroll
    for (int r = 0; r < R; ++r) fetch_one<KIND, R, NT>(o, r < nvalid ? T[r] : T[0], t, lane, f, r);
}

// Consume one fetched step: acc[r] += this lane's partial dot, in units of
// 2^-E (slots fetched for aliased tiles accumulate junk the caller drops).
// A(tau) yields this lane's A operand of x-image tile tau.
template <int KIND, int R, class ASrc>
__device__ __forceinline__ void compute_step(const Frag<KIND, R>& f, uint32_t t, const ASrc& A, const float* SX,
                                             int q, float* acc) {
    v4i c[R];
    if constexpr (KIND == HK_BIN) {
#pragma unroll
        for (int r = 0; r < R; ++r) c[r] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const v4i a = A(t * 8 + p);
            const uint32_t m = p < 7 ? 0x01010101u << p : 0xFFFFFFFFu;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const v4i b = p < 7 ? v4i{(int)(f.v[r].x & m), (int)(f.v[r].y & m), (int)(f.v[r].z & m), (int)(f.v[r].w & m)}
                                    : v4i{(int)f.v[r].x, (int)f.v[r].y, (int)f.v[r].z, (int)f.v[r].w};
                c[r] = mfma_i8(a, b, c[r]);
            }
        }
        const float2 u = reinterpret_cast<const float2*>(SX)[4 * t + q];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += f16_bits_to_f32(f.s[r]) * (combine_limbs(c[r]) * u.x - u.y);
    } else if constexpr (KIND == HK_Q4) {
        const uint32_t m = 0x0F0F0F0Fu;
        const v4i alo = A(t * 2), ahi = A(t * 2 + 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const v4i lo = {(int)(f.v[r].x & m), (int)(f.v[r].y & m), (int)(f.v[r].z & m), (int)(f.v[r].w & m)};
            const v4i hi = {(int)((f.v[r].x >> 4) & m), (int)((f.v[r].y >> 4) & m), (int)((f.v[r].z >> 4) & m),
                            (int)((f.v[r].w >> 4) & m)};
            c[r] = mfma_i8(alo, lo, v4i{0, 0, 0, 0});
            c[r] = mfma_i8(ahi, hi, c[r]);
        }
        const float2 u = reinterpret_cast<const float2*>(SX)[4 * t + q];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += f16_bits_to_f32(f.s[r]) * (combine_limbs(c[r]) * u.x - u.y);
    } else if constexpr (KIND == HK_Q8) {
        // code - 127 = (code ^ 0x80 as a signed byte) + 1: the B bytes are the
        // codes with the top bit flipped and the +1 is the slot's sum of X
        const v4i a = A(t);
        const uint32_t m = 0x80808080u;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const v4i b = {(int)(f.v[r].x ^ m), (int)(f.v[r].y ^ m), (int)(f.v[r].z ^ m), (int)(f.v[r].w ^ m)};
            c[r] = mfma_i8(a, b, v4i{0, 0, 0, 0});
        }
        const float2 u = reinterpret_cast<const float2*>(SX)[4 * t + q];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += f16_bits_to_f32(f.s[r]) * (combine_limbs(c[r]) * u.x - u.y);
    } else if constexpr (KIND == HK_U3) {
#pragma unroll
        for (int r = 0; r < R; ++r) c[r] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int mu = 0; mu < 4; ++mu) {
            const v4i a = A(t * 4 + mu);
            const uint32_t m2 = 0x03030303u << (2 * mu), m1 = 0x01010101u << (2 * mu);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t l0 = mu < 3 ? (f.lo[r].x & m2) : ((f.lo[r].x >> 6) & 0x03030303u);
                const uint32_t l1 = mu < 3 ? (f.lo[r].y & m2) : ((f.lo[r].y >> 6) & 0x03030303u);
                const v4i b = {(int)l0, (int)l1, (int)(f.hi[r] & m1), (int)(f.hi[r] & (m1 << 1))};
                c[r] = mfma_i8(a, b, c[r]);
            }
        }
        const float2 u = reinterpret_cast<const float2*>(SX)[4 * t + q];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += f16_bits_to_f32(f.s[r]) * (combine_limbs(c[r]) * u.x - u.y);
    } else {
        // field u of a byte is bits 2u..2u+1 (binary: bit 2u; the odd bits come
        // from the copy shifted down by one).  A Q2 item's bit 7 is stored
        // inverted, so its top field read as a signed byte is 64 (code - 2);
        // the x image's second sum corrects for that.
        uint32_t V[R][8];
        bool q2[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            q2[r] = __builtin_amdgcn_inverse_ballot_w64(f.q2m[r]);
            const uint32_t sh = q2[r] ? 0u : 1u;  // binary: odd columns are the signs >> 1
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                V[r][k] = f.V[r][k];
                V[r][k + 4] = f.V[r][k + 4] >> sh;
            }
        }
        // per half: {binary alpha, binary correction, Q2 alpha, Q2 correction};
        // each lane reads the pair of its kind
        float2 uh[2][R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float2* u2 = reinterpret_cast<const float2*>(SX) + 4 * (4 * t + q) + (q2[r] ? 1 : 0);
            uh[0][r] = u2[0];
            uh[1][r] = u2[2];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int r = 0; r < R; ++r) c[r] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const v4i a = A(t * 8 + h * 4 + u);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t bm = (q2[r] ? 0x03030303u : 0x01010101u) << (2 * u);
                    v4i b;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int ai = k < 2 ? 2 * h + k : 2 * h + 2 + k;
                        b[k] = (int)(V[r][ai] & bm);
                    }
                    c[r] = mfma_i8(a, b, c[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
                acc[r] += f16_bits_to_f32(h ? f.s1[r] : f.s0[r]) * (combine_limbs(c[r]) * uh[h][r].x - uh[h][r].y);
        }
    }
}

// Sum the four column-slot partials of a tile: every lane gets its row's total.
// v_permlane16_swap(v, v) leaves rows {0,0,2,2} in one result and {1,1,3,3}
// in the other (rows of 16 lanes), so their sum is v + v[lane ^ 16]; the
// 32-lane swap does the same for lane ^ 32.  Same bits as two xor shuffles.
__device__ __forceinline__ float tile_row_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

}  // namespace hk
