// Tiled weight layout shared by the host repack, the device repack and the
// kernels. One definition so every producer and consumer agree byte for byte.
//
// Geometry: rows in tiles of 16 (kTileRows); blocks of 32 elements in groups
// of 4 (kGroupBlocks, 128 k per group). A (tile, group) pair is one 64-lane
// wave's work unit: lane L = n + 16*kq (n = row in tile, kq = quarter 0..3)
// owns elements 8*kq .. 8*kq+7 of each of the group's 4 blocks of row n.
// That is exactly the B-operand fragment of v_mfma_f32_16x16x32_f16 when one
// MFMA covers one block (k = 32), so a block's fp16 scale can be applied to
// the MFMA result and every code is decoded exactly.
//
//  q4 quants: 16 B per lane, lane L of (t, g) at ((t*G + g)*64 + L)*16;
//             32-bit word w of the chunk = quarter kq of block 4g + w;
//             inside a word element 8*kq + i sits at nibble i/2 + 4*(i%2).
//  q8 quants: 2 x 16 B per lane at (((t*G + g)*2 + h)*64 + L)*16; chunk h,
//             words 2u and 2u+1 = quarter kq of block 4g + 2h + u
//             (elements 8kq..8kq+3 and 8kq+4..8kq+7); codes stored as q+128;
//             inside a word element 4w+i sits at byte i/2 + 2*(i%2).
//  scales d:  fp16 at index ((t*G + g)*16 + n)*4 + j for block 4g + j of row
//             16t + n (a lane reads its 4 scales as one 8-byte load).
//  mins m:    same indexing (q4_1 only).
// Rows past n and blocks past ceil(k/32) are padding that decodes to 0.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "mlq.h"

#if defined(__HIP__) || defined(__HIPCC__)
#define MLQ_HD __host__ __device__
#else
#define MLQ_HD
#endif

namespace mlq {

constexpr int kQK = 32;           // elements per GGUF block
constexpr int kTileRows = 16;     // rows per tile (MFMA n dimension)
constexpr int kGroupBlocks = 4;   // blocks per group (128 k)
constexpr int kGroupK = kQK * kGroupBlocks;
constexpr int kLanes = 64;        // lanes per (tile, group) = one wave
constexpr uint64_t kRegionAlign = 256;

struct Geometry {
  int n, k, nb, nt, g;  // rows, cols, blocks/row, row tiles, block groups
};

MLQ_HD inline Geometry geometry(int n, int k) {
  Geometry geo;
  geo.n = n;
  geo.k = k;
  geo.nb = (k + kQK - 1) / kQK;
  geo.nt = (n + kTileRows - 1) / kTileRows;
  geo.g = (geo.nb + kGroupBlocks - 1) / kGroupBlocks;
  return geo;
}

MLQ_HD inline uint64_t align_up(uint64_t v, uint64_t a) {
  return (v + a - 1) / a * a;
}

// Quant bytes per (tile, group, lane): one or two 16-byte chunks.
MLQ_HD inline int quant_bytes_per_lane(int type) {
  return type == MLQ_Q8_0 ? 32 : 16;
}

// (tile, group) units in the weight.
MLQ_HD inline uint64_t unit_count(const Geometry& geo) {
  return (uint64_t)geo.nt * geo.g;
}

// Scale/min entries (one per padded block).
MLQ_HD inline uint64_t scale_count(const Geometry& geo) {
  return unit_count(geo) * kTileRows * kGroupBlocks;
}

// Bit position (nibble index 0..7) of element i (0..7) inside a q4 word.
MLQ_HD inline int q4_nibble_in_word(int i) { return (i >> 1) + 4 * (i & 1); }

// Byte position (0..3) of element i (0..3) inside a q8 word.
MLQ_HD inline int q8_byte_in_word(int i) { return (i >> 1) + 2 * (i & 1); }

// Where element e (0..31) of block b of row `row` lives.
struct QuantPos {
  uint64_t byte;  // byte offset inside the quant region
  int shift;      // q4: 0 (low nibble) or 4 (high nibble); q8: 0
};

MLQ_HD inline QuantPos quant_pos(int type, const Geometry& geo, int row, int b,
                                 int e) {
  const int t = row / kTileRows, n = row % kTileRows;
  const int gi = b / kGroupBlocks, j = b % kGroupBlocks;
  const int kq = e >> 3, i = e & 7;
  const uint64_t unit = (uint64_t)t * geo.g + gi;
  const int lane = n + kTileRows * kq;
  QuantPos p;
  if (type == MLQ_Q8_0) {
    const int h = j >> 1, u = j & 1;
    const int word = 2 * u + (i >> 2);
    p.byte = ((unit * 2 + h) * kLanes + lane) * 16 + word * 4 +
             q8_byte_in_word(i & 3);
    p.shift = 0;
  } else {
    const int nib = q4_nibble_in_word(i);
    p.byte = (unit * kLanes + lane) * 16 + j * 4 + (nib >> 1);
    p.shift = (nib & 1) * 4;
  }
  return p;
}

// Index of the scale (and min) of block b of row `row`.
MLQ_HD inline uint64_t scale_index(const Geometry& geo, int row, int b) {
  const int t = row / kTileRows, n = row % kTileRows;
  const int gi = b / kGroupBlocks, j = b % kGroupBlocks;
  return (((uint64_t)t * geo.g + gi) * kTileRows + n) * kGroupBlocks + j;
}

}  // namespace mlq

namespace mlq {

// Writes one GGUF block (or, with src == nullptr, a padding block that
// decodes to 0) into the tiled layout. Shared by the host repack and the
// device repack kernel; each call owns every byte it writes, so blocks can
// be written in parallel.
MLQ_HD inline void repack_block(int type, const Geometry& geo, int row, int b,
                                const uint8_t* src, uint8_t* qs, uint16_t* d,
                                uint16_t* m) {
  const int t = row / kTileRows, n = row % kTileRows;
  const int gi = b / kGroupBlocks, j = b % kGroupBlocks;
  const uint64_t unit = (uint64_t)t * geo.g + gi;
  const uint64_t si = scale_index(geo, row, b);
  if (type == MLQ_Q8_0) {
    const int h = j >> 1, u = j & 1;
    for (int kq = 0; kq < 4; ++kq) {
      const int lane = n + kTileRows * kq;
      for (int hw = 0; hw < 2; ++hw) {
        uint32_t word = 0;
        for (int i = 0; i < 4; ++i) {
          const int e = 8 * kq + 4 * hw + i;
          const uint8_t q = src ? src[2 + e] : 0;  // int8 code
          word |= (uint32_t)(uint8_t)(q ^ 0x80u) << (8 * q8_byte_in_word(i));
        }
        uint8_t* dst = qs + ((unit * 2 + h) * kLanes + lane) * 16 + (2 * u + hw) * 4;
        dst[0] = (uint8_t)word;
        dst[1] = (uint8_t)(word >> 8);
        dst[2] = (uint8_t)(word >> 16);
        dst[3] = (uint8_t)(word >> 24);
      }
    }
    d[si] = src ? (uint16_t)(src[0] | (src[1] << 8)) : 0;
  } else {
    const int qoff = type == MLQ_Q4_0 ? 2 : 4;
    const uint8_t pad = type == MLQ_Q4_0 ? 8 : 0;  // code that decodes to 0
    for (int kq = 0; kq < 4; ++kq) {
      const int lane = n + kTileRows * kq;
      uint32_t word = 0;
      for (int i = 0; i < 8; ++i) {
        const int e = 8 * kq + i;
        uint8_t c = pad;
        if (src) {
          const uint8_t byte = src[qoff + (e & 15)];
          c = e < 16 ? (byte & 0x0f) : (byte >> 4);
        }
        word |= (uint32_t)c << (4 * q4_nibble_in_word(i));
      }
      uint8_t* dst = qs + (unit * kLanes + lane) * 16 + j * 4;
      dst[0] = (uint8_t)word;
      dst[1] = (uint8_t)(word >> 8);
      dst[2] = (uint8_t)(word >> 16);
      dst[3] = (uint8_t)(word >> 24);
    }
    d[si] = src ? (uint16_t)(src[0] | (src[1] << 8)) : 0;
    if (type == MLQ_Q4_1) m[si] = src ? (uint16_t)(src[2] | (src[3] << 8)) : 0;
  }
}

// Code of element e of block b of row `row` as stored (q8: signed q;
// q4: nibble 0..15).
MLQ_HD inline int read_code(int type, const Geometry& geo, const uint8_t* qs,
                            int row, int b, int e) {
  const QuantPos p = quant_pos(type, geo, row, b, e);
  if (type == MLQ_Q8_0) return (int)(int8_t)(qs[p.byte] ^ 0x80u);
  return (qs[p.byte] >> p.shift) & 0x0f;
}

}  // namespace mlq
