// hk_tile.h -- the wavefront-tiled device layout of packed organs.
//
// Rows are grouped in tiles of 16 (one MFMA N block); a tile is consumed in
// "steps", and one step is exactly one 1 KiB wave load: lane l of the wave
// (n = l % 16 = row in the tile, q = l / 16 = column slot) reads 16 bytes at
// offset 16*l.  Rows and columns are zero-padded to whole tiles and steps
// (zero scales contribute exactly 0).
//
//   BIN   step = 512 columns; lane (n,q) holds the 16 sign bytes of row n,
//         128-group 4t+q (bit i of byte j = column 8j+i, 1 = +scale).
//         scales: [tile][step][lane] f16 (one 128-byte line per step).
//   Q4    step = 128 columns; lane (n,q) holds the 16 code bytes of row n,
//         32-column chunk 4t+q (byte b: column 2b in the low nibble, 2b+1 in
//         the high nibble, value (nibble-8)*scale).
//         scales: [tile][step][lane] f16, the scale of the chunk's group
//         (duplicated per chunk when group > 32).
//   MIXED step = 512 columns; item (n,q) is row n, 128-group 4t+q, either
//         binary (16 B of signs, one f16 scale) or Q2 (32 B of 2-bit codes,
//         two f16 scales for columns 0-63 and 64-127).  Per (tile, step) a
//         16-byte header {q2mask.lo, q2mask.hi, data_off, scale_off}: item l
//         starts at data_off + 16*(l + popcount(q2mask below l)) bytes.  The
//         step's scales start at u16 scale_off (even): first the Q2 items'
//         pairs in lane order (Q2 lane l's pair at scale_off + 2 q, q =
//         popcount(q2mask below l)), then one scale per binary lane (lane l at
//         scale_off + 2 nq2 + l - q, nq2 = popcount(q2mask)), padded to whole
//         4-byte words, so every lane reads its scales with one aligned 4-byte
//         load (a binary lane takes the half of the word that holds its own).
//         Q2 code order inside an item (so one shift pattern decodes both
//         kinds): dword a (0..3) byte j holds, in 2-bit fields u = 0..3, the
//         codes of columns 32a + 8j + 2u; dword 4+a byte j holds columns
//         32a + 8j + 2u + 1.  Bit 7 of every Q2 byte is stored inverted, so
//         the top field read as a signed byte (bytes & 0xC0) is 64 (code - 2).
//   Q8    step = 64 columns (one group); lane (n,q) holds the 16 code bytes
//         of row n, columns 16q..16q+15 of the step (value (code-127)*scale).
//         scales: [tile][step][row] f16 (32 bytes per step: the four lanes of
//         a row read one scale, no duplication).
//   U3    step = 128 columns, 768 bytes: lane (n,q) holds row n, 32-column
//         chunk 4t+q as 12 bytes at 12*l: two dwords of the codes' low 2-bit
//         fields (column k of the chunk at bits 2(k%16) of dword k/16), then a
//         dword of their high bits (column k at bit k), one 12-byte load a
//         lane; nq = 4 column slots per step.  The last step
//         stores only the tail_q slots that hold columns (nq = tail_q), so a
//         narrow factor (cols = 160) carries no padded slots; lanes of absent
//         slots read slot 0's bytes (the x image is zero there).  Value
//         (lo + 4 hi - 3) * scale; scales: [tile][step][lane] f16 over the
//         stored lanes (the scale of the flat 64-group holding the chunk).
#pragma once

#include "hk_internal.h"

namespace hk {

constexpr uint32_t TILE_ROWS = 16;

// U3 bytes of one tile's data and scales (steps S, tail slots nql).
__host__ __device__ inline size_t u3_tile_data(uint32_t S, uint32_t nql) { return 768u * (size_t)(S - 1) + 192u * nql; }
__host__ __device__ inline size_t u3_tile_scales(uint32_t S, uint32_t nql) { return 64u * (size_t)(S - 1) + 16u * nql; }
__host__ __device__ inline uint32_t u3_tail_q(uint32_t cols) { return ((cols - 1u) % 128u) / 32u + 1u; }

__host__ __device__ inline uint32_t tile_step_cols(int kind) {
    return (kind == HK_Q4 || kind == HK_U3) ? 128u : kind == HK_Q8 ? 64u : 512u;
}
__host__ __device__ inline uint32_t n_tiles_for(uint32_t rows) { return (rows + TILE_ROWS - 1) / TILE_ROWS; }
__host__ __device__ inline uint32_t n_steps_for(int kind, uint32_t cols) {
    const uint32_t sc = tile_step_cols(kind);
    return (cols + sc - 1) / sc;
}

// Column (within the 128-group) of field u of byte j of dword a of a Q2 item.
__host__ __device__ inline uint32_t mixed_q2_col(uint32_t a, uint32_t j, uint32_t u) {
    return 32u * (a & 3u) + 8u * j + 2u * u + (a >> 2);
}

// Decoded weight (r, c) of a tiled organ, bit-exact with the reference
// decoders: (nibble-8)*scale, +-scale, (code-1.5)*scale.
__device__ inline float tiled_weight(const OrganView& o, uint32_t r, uint32_t c) {
    const uint32_t T = r / TILE_ROWS, n = r % TILE_ROWS;
    if (o.kind == HK_F32) return o.dense[(size_t)r * o.cols + c];
    if (o.kind == HK_Q4) {
        const uint32_t chunk = c >> 5, t = chunk >> 2, q = chunk & 3u, l = n + 16u * q, w = c & 31u;
        const uint8_t b = o.data[((size_t)T * o.steps + t) * 1024u + 16u * l + (w >> 1)];
        const int nib = (w & 1u) ? (b >> 4) : (b & 0xF);
        const float s = f16_bits_to_f32(o.scales[((size_t)T * o.steps + t) * 64u + l]);
        return (float)(nib - 8) * s;
    }
    if (o.kind == HK_U3) {
        const uint32_t t = c >> 7, q = (c >> 5) & 3u, k = c & 31u, l = n + 16u * q;
        const uint32_t nq = t + 1 == o.steps ? o.tail_q : 4u;
        const uint8_t* base = o.data + (size_t)T * u3_tile_data(o.steps, o.tail_q) + 768u * t;
        (void)nq;
        const uint32_t lo = *reinterpret_cast<const uint32_t*>(base + 12u * l + 4u * (k >> 4));
        const uint32_t hi = *reinterpret_cast<const uint32_t*>(base + 12u * l + 8u);
        const uint32_t code = ((lo >> (2u * (k & 15u))) & 3u) + 4u * ((hi >> k) & 1u);
        const float s = f16_bits_to_f32(o.scales[(size_t)T * u3_tile_scales(o.steps, o.tail_q) + 64u * t + l]);
        return (float)((int)code - 3) * s;
    }
    if (o.kind == HK_Q8) {
        const uint32_t t = c >> 6, q = (c >> 4) & 3u, l = n + 16u * q;
        const uint8_t b = o.data[((size_t)T * o.steps + t) * 1024u + 16u * l + (c & 15u)];
        const float s = f16_bits_to_f32(o.scales[((size_t)T * o.steps + t) * 16u + n]);
        return (float)((int)b - 127) * s;
    }
    const uint32_t g = c >> 7, t = g >> 2, q = g & 3u, l = n + 16u * q, i = c & 127u;
    if (o.kind == HK_BIN) {
        const uint8_t b = o.data[((size_t)T * o.steps + t) * 1024u + 16u * l + (i >> 3)];
        const float s = f16_bits_to_f32(o.scales[((size_t)T * o.steps + t) * 64u + l]);
        return ((b >> (i & 7u)) & 1u) ? s : -s;
    }
    const uint4 h = o.hdr[(size_t)T * o.steps + t];
    const uint64_t mask = (uint64_t)h.x | ((uint64_t)h.y << 32);
    const uint32_t below = __popcll(mask & ((1ull << l) - 1ull)), nq2 = __popcll(mask);
    const uint8_t* item = o.data + h.z + 16u * (l + below);
    const bool q2 = (mask >> l) & 1ull;
    const uint16_t* sc = o.scales + h.w + (q2 ? 2u * below : 2u * nq2 + l - below);
    if (!q2) {
        const float s = f16_bits_to_f32(sc[0]);
        return ((item[i >> 3] >> (i & 7u)) & 1u) ? s : -s;
    }
    // invert mixed_q2_col: column i -> (a, j, u)
    const uint32_t a = ((i >> 5) & 3u) | ((i & 1u) << 2), j = (i >> 3) & 3u, u = (i >> 1) & 3u;
    const uint32_t code = ((item[4u * a + j] ^ 0x80u) >> (2u * u)) & 3u;  // bit 7 is stored inverted
    return ((float)code - 1.5f) * f16_bits_to_f32(sc[i >> 6]);
}

}  // namespace hk
