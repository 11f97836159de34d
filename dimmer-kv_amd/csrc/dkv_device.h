// Device-side helpers shared by the Dimmer-KV HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dimmerkv.h"

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define DKV_DEVICE __device__ __forceinline__

// 32-bit rotate right by a compile-time amount.
DKV_DEVICE uint32_t rotr32(uint32_t x, int s) { return s == 0 ? x : ((x >> s) | (x << (32 - s))); }

DKV_DEVICE float half_bits_to_float(uint16_t h) {
  half_t v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

DKV_DEVICE float bf16_bits_to_float(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Round-to-nearest-even float -> bf16 bits.
DKV_DEVICE uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

DKV_DEVICE float load_as_float(const void* p, long idx, int dtype) {
  if (dtype == DKV_F32) return ((const float*)p)[idx];
  if (dtype == DKV_F16) return half_bits_to_float(((const uint16_t*)p)[idx]);
  return bf16_bits_to_float(((const uint16_t*)p)[idx]);
}

DKV_DEVICE void store_from_float(void* p, long idx, int dtype, float v) {
  if (dtype == DKV_F32) {
    ((float*)p)[idx] = v;
  } else if (dtype == DKV_F16) {
    half_t h = (half_t)v;
    uint16_t bits;
    __builtin_memcpy(&bits, &h, 2);
    ((uint16_t*)p)[idx] = bits;
  } else {
    ((uint16_t*)p)[idx] = float_to_bf16_bits(v);
  }
}

// ---------------------------------------------------------------------------
// Bit-plane unpack.
//
// A plane word is two u32 halves; half h holds coefficients 32h..32h+31.
// Coefficient 32h + 4w + i (w in 0..7, i in 0..3) of plane p is stored at bit
// (8i + w + 7 - p) mod 32 and carries bit (7 - p) of the coefficient's 8-bit
// code.  Given the (up to 8) plane halves of one (token, group, half), the
// code word w (four codes, byte i = coefficient 4w+i, truncated to the
// present planes with the missing low bits 0) is
//     rotr( OR_p  plane[p] & (0x01010101 << ((w + 7 - p) & 7)),  w ).
// Absent planes are passed as 0.
// ---------------------------------------------------------------------------
template <int W>
DKV_DEVICE uint32_t assemble_codes(const uint32_t (&pl)[8]) {
  uint32_t acc = 0;
#pragma unroll
  for (int p = 0; p < 8; ++p) acc |= pl[p] & (0x01010101u << ((W + 7 - p) & 7));
  return rotr32(acc, W);
}

// Loads the header and plane halves of one (token, group, half).
// seg points at the group's hot segment ([low f16][span f16][m words]).
DKV_DEVICE void load_segment(const uint8_t* seg, int m, int half, uint32_t (&pl)[8], uint32_t& header) {
  const uint32_t* w = (const uint32_t*)seg;
  header = (m > 0) ? w[0] : 0u;
#pragma unroll
  for (int p = 0; p < 8; ++p) pl[p] = (p < m) ? w[1 + 2 * p + half] : 0u;
}

// Branch-free variant: absent planes (and the whole segment when m == 0) read
// from ``safe`` (any valid address) and are then zeroed.
DKV_DEVICE void load_segment_nb(const uint8_t* seg, int m, int half, const uint8_t* safe, uint32_t (&pl)[8],
                                uint32_t& header) {
  const uint32_t* w = (const uint32_t*)(m > 0 ? seg : safe);
  const uint32_t* sw = (const uint32_t*)safe;
  const uint32_t h = w[0];
  header = m > 0 ? h : 0u;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const uint32_t v = *((p < m) ? (w + 1 + 2 * p + half) : sw);
    pl[p] = (p < m) ? v : 0u;
  }
}

// Dequantized value in the reference's exact fp32 operation order
// (scripts/progressive.py:53): low + ((idx + 0.5) * span) / 2^m, every
// product and sum rounded on its own; m == 0 gives 0.
DKV_DEVICE float dequant_exact(uint32_t code8, int m, float low, float span, float inv_bins) {
#pragma clang fp contract(off)
  if (m == 0) return 0.0f;
  const uint32_t idx = code8 >> (8 - m);
  const float prod = ((float)idx + 0.5f) * span;
  return low + prod * inv_bins;  // * 2^-m is exact, equal to / 2^m
}

// Per-(token, group) affine form used to feed MFMA operands:
// value = code8 * scale + offset  with scale = span/256, offset = low + span*2^-(m+1)
// (equal to the exact form up to one fp32 rounding; the result is then
// rounded to fp16 anyway).
struct AffineDq {
  float scale, offset;
};

DKV_DEVICE AffineDq affine_from_header(uint32_t header, int m) {
  AffineDq a;
  if (m == 0) {
    a.scale = 0.0f;
    a.offset = 0.0f;
  } else {
    const float low = half_bits_to_float((uint16_t)(header & 0xffffu));
    const float span = half_bits_to_float((uint16_t)(header >> 16));
    a.scale = span * (1.0f / 256.0f);
    a.offset = low + span * __builtin_ldexpf(1.0f, -(m + 1));
  }
  return a;
}

// 32 codes of one (token, group, half) -> 32 fp16 values (affine form),
// stored as 16 packed half2 words in out[0..15] (element j = coefficient j).
DKV_DEVICE void unpack_half_f16(const uint32_t (&pl)[8], AffineDq a, uint32_t (&out)[16]) {
  uint32_t cw[8];
  cw[0] = assemble_codes<0>(pl);
  cw[1] = assemble_codes<1>(pl);
  cw[2] = assemble_codes<2>(pl);
  cw[3] = assemble_codes<3>(pl);
  cw[4] = assemble_codes<4>(pl);
  cw[5] = assemble_codes<5>(pl);
  cw[6] = assemble_codes<6>(pl);
  cw[7] = assemble_codes<7>(pl);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const uint32_t c = cw[w];
    const float v0 = __builtin_fmaf((float)(c & 0xffu), a.scale, a.offset);
    const float v1 = __builtin_fmaf((float)((c >> 8) & 0xffu), a.scale, a.offset);
    const float v2 = __builtin_fmaf((float)((c >> 16) & 0xffu), a.scale, a.offset);
    const float v3 = __builtin_fmaf((float)(c >> 24), a.scale, a.offset);
    half_t h0 = (half_t)v0, h1 = (half_t)v1, h2 = (half_t)v2, h3 = (half_t)v3;
    uint16_t b0, b1, b2, b3;
    __builtin_memcpy(&b0, &h0, 2);
    __builtin_memcpy(&b1, &h1, 2);
    __builtin_memcpy(&b2, &h2, 2);
    __builtin_memcpy(&b3, &h3, 2);
    out[2 * w] = (uint32_t)b0 | ((uint32_t)b1 << 16);
    out[2 * w + 1] = (uint32_t)b2 | ((uint32_t)b3 << 16);
  }
}

// ---------------------------------------------------------------------------
// kvtc ladder codes.  A (token, group) segment with b in {2, 4, 8} bits is
// [low f16][scale f16][64 codes of b bits, LSB-first]; the codes of half h
// (coefficients 32h .. 32h+31) are the b u32 words starting at byte 4 + 4bh.
// They are returned in the plane path's code-word form: byte i of cw[w] is the
// code of coefficient 32h + 4w + i.  b = 0 gives zero codes and header.
// ---------------------------------------------------------------------------
DKV_DEVICE int dkv_groups(const dkv_stream_t& s) {
  return s.format == DKV_FMT_LADDER ? s.ladder.groups : s.order.groups;
}

DKV_DEVICE uint32_t spread_nibbles(uint32_t x) {  // 4 nibbles (16 bits) -> 4 bytes
  return (x & 0xfu) | ((x & 0xf0u) << 4) | ((x & 0xf00u) << 8) | ((x & 0xf000u) << 12);
}

DKV_DEVICE uint32_t spread_pairs(uint32_t x) {  // 4 two-bit fields (8 bits) -> 4 bytes
  return (x & 0x3u) | ((x & 0xcu) << 6) | ((x & 0x30u) << 12) | ((x & 0xc0u) << 18);
}

// The b packed words of one half (raw[k], k < b; the rest ignored) -> the code-word form.
DKV_DEVICE void ladder_half_codes(const uint32_t (&raw)[8], int b, uint32_t (&cw)[8]) {
  if (b == 4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      cw[2 * k] = spread_nibbles(raw[k] & 0xffffu);
      cw[2 * k + 1] = spread_nibbles(raw[k] >> 16);
    }
  } else if (b == 2) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) cw[4 * k + j] = spread_pairs((raw[k] >> (8 * j)) & 0xffu);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) cw[k] = raw[k];  // b == 8 (b == 0: all zero)
  }
}

DKV_DEVICE void load_ladder_half(const uint8_t* seg, int b, int half, uint32_t (&cw)[8], uint32_t& header) {
  const uint32_t* w = (const uint32_t*)seg;
  header = b > 0 ? w[0] : 0u;
  const uint32_t* c = w + 1 + b * half;
  uint32_t raw[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) raw[k] = k < b ? c[k] : 0u;
  ladder_half_codes(raw, b, cw);
}

// A whole (token, group) segment: the header word and its first nwords code words (nwords even,
// at most 16; the rest 0), read with one 16-byte load per four words (two for a final pair).
// Plane segments hold word 2p + h = half h of plane p (nwords = 2m).  Segments are 4-byte aligned,
// which the multi-word global loads accept.
DKV_DEVICE void load_segment_words(const uint8_t* seg, int nwords, uint32_t& header, uint32_t (&w)[16]) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const uint32_t* p = (const uint32_t*)seg;
  header = nwords > 0 ? p[0] : 0u;
  // full pieces and the final pair load into registers of their own and meet in selects after
  // the loads, so no load waits for another (a shared destination would order them)
  u32x4 v[4];
  u32x2 tail = {0u, 0u};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = u32x4{0u, 0u, 0u, 0u};
    if (4 * k + 4 <= nwords) __builtin_memcpy(&v[k], p + 1 + 4 * k, 16);
  }
  const int kt = nwords >> 2;  // the piece holding a final pair (nwords % 4 == 2)
  if (nwords & 2) __builtin_memcpy(&tail, p + 1 + 4 * kt, 8);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const bool pair = (nwords & 2) && k == kt;
    w[4 * k] = pair ? tail.x : v[k].x;
    w[4 * k + 1] = pair ? tail.y : v[k].y;
    w[4 * k + 2] = v[k].z;
    w[4 * k + 3] = v[k].w;
  }
}

// A whole ladder segment with b bits (0, 2, 4 or 8): the header word, half h's b words in
// w[8h .. 8h+b-1] (the rest 0).  Each half is read from its own address (word 1 + b h), so the
// registers it lands in do not depend on b.
DKV_DEVICE void load_ladder_segment(const uint8_t* seg, int b, uint32_t& header, uint32_t (&w)[16]) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const uint32_t* p = (const uint32_t*)seg;
  header = b > 0 ? p[0] : 0u;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t* base = p + 1 + b * h;
    u32x4 v0 = {0u, 0u, 0u, 0u}, v1 = {0u, 0u, 0u, 0u};
    u32x2 pair = {0u, 0u};
    if (b >= 4) __builtin_memcpy(&v0, base, 16);
    if (b == 8) __builtin_memcpy(&v1, base + 4, 16);
    if (b == 2) __builtin_memcpy(&pair, base, 8);
    w[8 * h + 0] = b == 2 ? pair.x : v0.x;
    w[8 * h + 1] = b == 2 ? pair.y : v0.y;
    w[8 * h + 2] = v0.z;
    w[8 * h + 3] = v0.w;
    w[8 * h + 4] = v1.x;
    w[8 * h + 5] = v1.y;
    w[8 * h + 6] = v1.z;
    w[8 * h + 7] = v1.w;
  }
}

// Half h (0 or 1) of a ladder segment loaded by load_ladder_segment, in the code-word form.
DKV_DEVICE void ladder_segment_half(const uint32_t (&w)[16], int b, int h, uint32_t (&cw)[8]) {
  uint32_t raw[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) raw[k] = w[8 * h + k];
  ladder_half_codes(raw, b, cw);
}

// Ladder coefficient in the reference's fp32 operation order
// (scripts/kvtc.py:78): code * scale + low, the product and the sum each
// rounded on its own.  A zero header (b = 0) gives 0.
DKV_DEVICE float ladder_value(uint32_t code, float low, float scale) {
#pragma clang fp contract(off)
  const float prod = (float)code * scale;
  return prod + low;
}

// 32 ladder codes of one (token, group, half) -> 32 fp16 values (the fp16
// cast of the exact fp32 coefficient), as 16 packed half2 words.
DKV_DEVICE void ladder_half_f16(const uint32_t (&cw)[8], uint32_t header, uint32_t (&out)[16]) {
  const float low = half_bits_to_float((uint16_t)(header & 0xffffu));
  const float scale = half_bits_to_float((uint16_t)(header >> 16));
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint16_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const half_t h = (half_t)ladder_value((cw[w] >> (8 * i)) & 0xffu, low, scale);
      __builtin_memcpy(&b[i], &h, 2);
    }
    out[2 * w] = (uint32_t)b[0] | ((uint32_t)b[1] << 16);
    out[2 * w + 1] = (uint32_t)b[2] | ((uint32_t)b[3] << 16);
  }
}

// Sequence/tile lookup from cu_seqlens without a host-built table: returns
// the sequence b and the tile index inside it for a global tile id, where
// sequence b has ceil(len_b / tile) tiles.  One sequence (n_total tokens)
// needs no load.
DKV_DEVICE int2 find_tile(const int32_t* cu, int batch, int n_total, int tile, int gid) {
  if (batch == 1) return make_int2(gid < (n_total + tile - 1) / tile ? 0 : -1, gid);
  int base = 0;
  for (int b = 0; b < batch; ++b) {
    const int len = cu[b + 1] - cu[b];
    const int nt = (len + tile - 1) / tile;
    if (gid < base + nt) return make_int2(b, gid - base);
    base += nt;
  }
  return make_int2(-1, 0);
}

// First and one-past-last token of sequence b.  With one sequence they are 0
// and n_total from the kernel arguments, so the first data loads do not wait
// on a load of cu_seqlens.
DKV_DEVICE int2 seq_range(const int32_t* cu, int batch, int n_total, int b) {
  return batch == 1 ? make_int2(0, n_total) : make_int2(cu[b], cu[b + 1]);
}

// ---------------------------------------------------------------------------
// Cross-lane steps on the VALU (DPP and gfx950's permlane swaps) instead of
// LDS-routed shuffles: each is a few cycles rather than an LDS round trip.
// The DPP forms: quad_perm [1,0,3,2] = lane ^ 1, quad_perm [2,3,0,1] = lane ^ 2,
// row_half_mirror = lane i <-> 7 - i within 8, row_mirror = i <-> 15 - i
// within 16.  After the two quad steps every lane of a quad holds the quad's
// reduction, so the mirrors then pair lanes of different quads (and halves of
// a row): the four steps reduce a row of 16.  The permlane swaps exchange rows
// (lane ^ 16) and wave halves (lane ^ 32); they return each lane's own value
// and its partner's in an order that depends on the row, so they serve only
// symmetric combinations (sum, max).
// ---------------------------------------------------------------------------
template <int CTRL>
DKV_DEVICE float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
DKV_DEVICE float lane_xor1(float v) { return dpp_f32<0xB1>(v); }
DKV_DEVICE float lane_xor2(float v) { return dpp_f32<0x4E>(v); }
DKV_DEVICE float lane_half_mirror(float v) { return dpp_f32<0x141>(v); }
DKV_DEVICE float lane_mirror(float v) { return dpp_f32<0x140>(v); }

DKV_DEVICE float sum_xor16(float v) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
DKV_DEVICE float max_xor16(float v) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
DKV_DEVICE float sum_xor32(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
DKV_DEVICE float max_xor32(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// Reductions over groups of 8, 16 and 32 consecutive lanes (every lane of a group gets the result).
DKV_DEVICE float max8(float v) {
  v = fmaxf(v, lane_xor1(v));
  v = fmaxf(v, lane_xor2(v));
  return fmaxf(v, lane_half_mirror(v));
}
DKV_DEVICE float sum8(float v) {
  v += lane_xor1(v);
  v += lane_xor2(v);
  return v + lane_half_mirror(v);
}
DKV_DEVICE float max16(float v) { v = max8(v); return fmaxf(v, lane_mirror(v)); }
DKV_DEVICE float sum16(float v) {
  v += lane_xor1(v);
  v += lane_xor2(v);
  v += lane_half_mirror(v);
  return v + lane_mirror(v);
}
DKV_DEVICE float max32(float v) { return max_xor16(max16(v)); }
DKV_DEVICE float sum32(float v) { return sum_xor16(sum16(v)); }

DKV_DEVICE float wave_max(float v) { return max_xor32(max32(v)); }
DKV_DEVICE float wave_sum(float v) { return sum_xor32(sum32(v)); }
