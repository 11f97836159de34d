// Packing, K1 unpack/dequantize, cold-plane gather (K4c) and basis layouts.
//
// Reference behaviour replaced here (SrikanthBalaaji/Dimmer-KV):
//   scripts/progressive.py:47-55   dequantize
//   scripts/progressive.py:103-110 TokenStore (codes kept unpacked; only counted)
//   scripts/progressive.py:185-194 hot/cold byte accounting
//   scripts/progressive.py:224-236 ProgressiveCache.refine (cold pieces of the top tokens)
#include <string>

#include "dkv_device.h"
#include "dkv_host.h"

namespace dkv {
static thread_local std::string g_error;
void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}
}  // namespace dkv

extern "C" int dkv_abi_version(void) { return DKV_ABI_VERSION; }
extern "C" const char* dkv_last_error(void) { return dkv::g_error.c_str(); }

// ---------------------------------------------------------------------------
// Pack: one wave per (token, group).  Lane L owns bit position L of each
// plane word; it fetches (by cross-lane shuffle) the code of the coefficient
// that the layout puts at that position and the wave ballots the bit.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_kernel(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ low,
                                                   const uint16_t* __restrict__ span,
                                                   const int16_t* __restrict__ pieces, int n, dkv_order_t order,
                                                   uint8_t* __restrict__ hot, const int64_t* __restrict__ hot_off,
                                                   uint8_t* __restrict__ cold,
                                                   const int64_t* __restrict__ cold_tok_off) {
  const int G = order.groups;
  const long gw = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (gw >= (long)n * G) return;
  const int t = (int)(gw / G), g = (int)(gw % G);
  const int k = pieces[t];
  const int m = order.planes[(long)k * G + g];
  const int m_full = order.planes[(long)order.pieces * G + g];
  const uint32_t code = codes[gw * 64 + lane];
  uint64_t words[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int jj = ((lane & 31) + 25 + p) & 31;  // (q - 7 + p) mod 32
    const int coef = (lane & 32) + 4 * (jj & 7) + (jj >> 3);
    const uint32_t c = (uint32_t)__shfl((int)code, coef, 64);
    words[p] = __ballot((c >> (7 - p)) & 1u);
  }
  const uint32_t header = (uint32_t)low[gw] | ((uint32_t)span[gw] << 16);
  if (m > 0) {
    uint32_t* dst = (uint32_t*)(hot + hot_off[t] + order.seg_off[(long)k * G + g]);
    if (lane == 0) dst[0] = header;
    if (lane < m) {
      uint64_t wv = 0;
#pragma unroll
      for (int p = 0; p < 8; ++p) wv = (p == lane) ? words[p] : wv;
      dst[1 + 2 * lane] = (uint32_t)wv;
      dst[2 + 2 * lane] = (uint32_t)(wv >> 32);
    }
  }
  if (cold != nullptr && m < m_full) {
    uint32_t* dst = (uint32_t*)(cold + cold_tok_off[t] + order.cold_off[(long)k * G + g]);
    if (m == 0) {
      if (lane == 0) dst[0] = header;
      dst += 1;
    }
    if (lane >= m && lane < m_full) {
      uint64_t wv = 0;
#pragma unroll
      for (int p = 0; p < 8; ++p) wv = (p == lane) ? words[p] : wv;
      dst[2 * (lane - m)] = (uint32_t)wv;
      dst[2 * (lane - m) + 1] = (uint32_t)(wv >> 32);
    }
  }
}

extern "C" int dkv_pack_planes(const uint8_t* codes, const uint16_t* low, const uint16_t* span, const int16_t* pieces,
                               int32_t n, dkv_order_t order, uint8_t* hot, const int64_t* hot_off, uint8_t* cold,
                               const int64_t* cold_off, void* stream) {
  DKV_REQUIRE(n >= 0, DKV_ESHAPE, "dkv_pack_planes: n < 0");
  int rc = dkv::check_order(order, "dkv_pack_planes");
  if (rc) return rc;
  if (n == 0) return DKV_OK;
  DKV_REQUIRE(codes && low && span && pieces && hot && hot_off, DKV_EINVAL, "dkv_pack_planes: null pointer");
  DKV_REQUIRE(!cold || (cold_off && order.cold_off), DKV_EINVAL, "dkv_pack_planes: cold needs cold offsets");
  const long waves = (long)n * order.groups;
  const long blocks = (waves + 3) / 4;
  DKV_REQUIRE(blocks < (1L << 31), DKV_ESHAPE, "dkv_pack_planes: too many tokens");
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, dkv::as_stream(stream), codes, low, span,
                     pieces, n, order, hot, hot_off, cold, cold_off);
  return dkv::check_launch("dkv_pack_planes");
}

// ---------------------------------------------------------------------------
// Ladder pack: one thread per (token, group, half).  The 32 codes of the half
// are squeezed to b bits each, LSB-first (code j at bit b*j), into b words;
// the thread of half 0 also writes the [low][scale] header.
// ---------------------------------------------------------------------------
DKV_DEVICE uint32_t gather_nibbles(uint32_t c) {  // 4 bytes < 16 -> 16 bits
  return (c & 0xfu) | ((c >> 4) & 0xf0u) | ((c >> 8) & 0xf00u) | ((c >> 12) & 0xf000u);
}

DKV_DEVICE uint32_t gather_pairs(uint32_t c) {  // 4 bytes < 4 -> 8 bits
  return (c & 0x3u) | ((c >> 6) & 0xcu) | ((c >> 12) & 0x30u) | ((c >> 18) & 0xc0u);
}

__global__ __launch_bounds__(256) void pack_ladder_kernel(const uint8_t* __restrict__ codes,
                                                          const uint16_t* __restrict__ low,
                                                          const uint16_t* __restrict__ scale,
                                                          const int16_t* __restrict__ rung, int n, dkv_ladder_t lad,
                                                          uint8_t* __restrict__ blob,
                                                          const int64_t* __restrict__ tok_off) {
  const int G = lad.groups;
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)n * G * 2) return;
  const int h = (int)(id & 1);
  const long tg = id >> 1;
  const int t = (int)(tg / G), g = (int)(tg % G);
  const int r = rung[t];
  if (r < 0 || r >= lad.rungs) return;
  const int b = lad.bits[(long)r * G + g];
  if (b != 2 && b != 4 && b != 8) return;
  uint32_t* seg = (uint32_t*)(blob + tok_off[t] + lad.seg_off[(long)r * G + g]);
  if (h == 0) seg[0] = (uint32_t)low[tg] | ((uint32_t)scale[tg] << 16);
  const uint4* src = (const uint4*)(codes + tg * 64 + h * 32);
  const uint4 c0 = src[0], c1 = src[1];
  const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  uint32_t* dst = seg + 1 + b * h;
  if (b == 8) {
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = cw[k];
  } else if (b == 4) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      dst[k] = gather_nibbles(cw[2 * k] & 0x0f0f0f0fu) | (gather_nibbles(cw[2 * k + 1] & 0x0f0f0f0fu) << 16);
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      uint32_t wv = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) wv |= gather_pairs(cw[4 * k + j] & 0x03030303u) << (8 * j);
      dst[k] = wv;
    }
  }
}

extern "C" int dkv_pack_ladder(const uint8_t* codes, const uint16_t* low, const uint16_t* scale, const int16_t* rung,
                               int32_t n, dkv_ladder_t ladder, uint8_t* blob, const int64_t* tok_off, void* stream) {
  DKV_REQUIRE(n >= 0, DKV_ESHAPE, "dkv_pack_ladder: n < 0");
  int rc = dkv::check_ladder(ladder, "dkv_pack_ladder");
  if (rc) return rc;
  if (n == 0) return DKV_OK;
  DKV_REQUIRE(codes && low && scale && rung && blob && tok_off, DKV_EINVAL, "dkv_pack_ladder: null pointer");
  const long threads = (long)n * ladder.groups * 2;
  const long blocks = (threads + 255) / 256;
  DKV_REQUIRE(blocks < (1L << 31), DKV_ESHAPE, "dkv_pack_ladder: too many tokens");
  hipLaunchKernelGGL(pack_ladder_kernel, dim3((unsigned)blocks), dim3(256), 0, dkv::as_stream(stream), codes, low,
                     scale, rung, n, ladder, blob, tok_off);
  return dkv::check_launch("dkv_pack_ladder");
}

// ---------------------------------------------------------------------------
// Byte storage.  One thread per (token, group, half): the half's 32 codes are
// 4b bytes of the (token, group)'s code run, which starts at a byte boundary
// (64 b-bit codes are 8b bytes), so halves never share a byte.  Storage
// positions carry no alignment (the sections follow byte-sized rung ids), so
// the storage side moves single bytes; the code/shift/scale side is aligned.
// ---------------------------------------------------------------------------
struct WireSpot {
  long code, low, scale;  // byte positions of the half's codes and of the group's shift and scale
  int b;                  // width, 0 = nothing to move
};

DKV_DEVICE int width_index(int b) { return b == 2 ? 0 : (b == 4 ? 1 : 2); }

DKV_DEVICE WireSpot wire_spot(const int16_t* __restrict__ rung, const dkv_ladder_t& lad, const dkv_wire_t& w, int t,
                              int g, int h) {
  WireSpot s{0, 0, 0, 0};
  const int G = lad.groups;
  const int r = rung[t];
  if (r < 0 || r >= lad.rungs) return s;
  const int b = lad.bits[(long)r * G + g];
  if (b != 2 && b != 4 && b != 8) return s;
  const int wi = width_index(b);
  const long cnt = w.count[r], nw = w.nwidth[3 * r + wi];
  const long k = w.rank[t], j = w.slot[(long)r * G + g];
  if (k < 0 || k >= cnt || j < 0 || j >= nw) return s;
  const long base = w.section[3 * r + wi];
  const long item = k * nw + j;
  s.code = base + item * 8 * b + 4 * b * h;
  s.low = base + cnt * nw * 8 * b + item * 2;
  s.scale = base + cnt * nw * (8 * b + 2) + item * 2;
  if (base < 0 || s.scale + 2 > w.bytes) return s;  // outside the storage buffer: leave it alone
  s.b = b;
  return s;
}

__global__ __launch_bounds__(256) void wire_pack_kernel(const uint8_t* __restrict__ codes,
                                                        const uint16_t* __restrict__ low,
                                                        const uint16_t* __restrict__ scale,
                                                        const int16_t* __restrict__ rung, int n, dkv_ladder_t lad,
                                                        dkv_wire_t w, uint8_t* __restrict__ out) {
  const int G = lad.groups;
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)n * G * 2) return;
  const int h = (int)(id & 1);
  const long tg = id >> 1;
  const int t = (int)(tg / G), g = (int)(tg % G);
  const WireSpot s = wire_spot(rung, lad, w, t, g, h);
  if (s.b == 0) return;
  const uint4* src = (const uint4*)(codes + tg * 64 + h * 32);
  const uint4 c0 = src[0], c1 = src[1];
  const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  uint32_t pw[8];
  if (s.b == 8) {
#pragma unroll
    for (int k = 0; k < 8; ++k) pw[k] = cw[k];
  } else if (s.b == 4) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      pw[k] = gather_nibbles(cw[2 * k] & 0x0f0f0f0fu) | (gather_nibbles(cw[2 * k + 1] & 0x0f0f0f0fu) << 16);
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      uint32_t wv = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) wv |= gather_pairs(cw[4 * k + j] & 0x03030303u) << (8 * j);
      pw[k] = wv;
    }
  }
  uint8_t* dst = out + s.code;
#pragma unroll
  for (int k = 0; k < 8; ++k)  // b words = 4b bytes
    if (k < s.b)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[4 * k + i] = (uint8_t)(pw[k] >> (8 * i));
  if (h == 0) {
    const uint16_t lo = low[tg], sc = scale[tg];
    out[s.low] = (uint8_t)lo;
    out[s.low + 1] = (uint8_t)(lo >> 8);
    out[s.scale] = (uint8_t)sc;
    out[s.scale + 1] = (uint8_t)(sc >> 8);
  }
}

// The 32 codes of a half from its 4B storage bytes (code i at bit B*i), one code per byte of cw.
template <int B>
DKV_DEVICE void wire_codes_half(const uint8_t* __restrict__ src, uint32_t (&cw)[8]) {
  uint32_t pw[B];
#pragma unroll
  for (int k = 0; k < B; ++k)
    pw[k] = (uint32_t)src[4 * k] | ((uint32_t)src[4 * k + 1] << 8) | ((uint32_t)src[4 * k + 2] << 16) |
            ((uint32_t)src[4 * k + 3] << 24);
  constexpr uint32_t kMask = (1u << B) - 1u;
#pragma unroll
  for (int k = 0; k < 8; ++k) {  // codes 4k .. 4k+3
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int bit = (4 * k + i) * B;
      v |= ((pw[bit >> 5] >> (bit & 31)) & kMask) << (8 * i);
    }
    cw[k] = v;
  }
}

__global__ __launch_bounds__(256) void wire_unpack_kernel(const uint8_t* __restrict__ in,
                                                          const int16_t* __restrict__ rung, int n, dkv_ladder_t lad,
                                                          dkv_wire_t w, uint8_t* __restrict__ codes,
                                                          uint16_t* __restrict__ low, uint16_t* __restrict__ scale) {
  const int G = lad.groups;
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)n * G * 2) return;
  const int h = (int)(id & 1);
  const long tg = id >> 1;
  const int t = (int)(tg / G), g = (int)(tg % G);
  const WireSpot s = wire_spot(rung, lad, w, t, g, h);
  if (s.b == 0) return;
  uint32_t cw[8];
  if (s.b == 8) {
    wire_codes_half<8>(in + s.code, cw);
  } else if (s.b == 4) {
    wire_codes_half<4>(in + s.code, cw);
  } else {
    wire_codes_half<2>(in + s.code, cw);
  }
  uint4* dst = (uint4*)(codes + tg * 64 + h * 32);
  dst[0] = make_uint4(cw[0], cw[1], cw[2], cw[3]);
  dst[1] = make_uint4(cw[4], cw[5], cw[6], cw[7]);
  if (h == 0) {
    low[tg] = (uint16_t)(in[s.low] | (in[s.low + 1] << 8));
    scale[tg] = (uint16_t)(in[s.scale] | (in[s.scale + 1] << 8));
  }
}

static int check_wire(const dkv_wire_t& w, int32_t n, const char* what) {
  if (!w.section || !w.count || !w.slot || !w.nwidth || (n > 0 && !w.rank) || w.bytes < 0) {
    dkv::set_error("%s: storage tables must be non-null and bytes >= 0", what);
    return DKV_EINVAL;
  }
  return DKV_OK;
}

extern "C" int dkv_wire_pack(const uint8_t* codes, const uint16_t* low, const uint16_t* scale, const int16_t* rung,
                             int32_t n, dkv_ladder_t ladder, dkv_wire_t wire, uint8_t* out, void* stream) {
  DKV_REQUIRE(n >= 0, DKV_ESHAPE, "dkv_wire_pack: n < 0");
  int rc = dkv::check_ladder(ladder, "dkv_wire_pack");
  if (rc) return rc;
  if ((rc = check_wire(wire, n, "dkv_wire_pack"))) return rc;
  if (n == 0) return DKV_OK;
  DKV_REQUIRE(codes && low && scale && rung && out, DKV_EINVAL, "dkv_wire_pack: null pointer");
  const long blocks = ((long)n * ladder.groups * 2 + 255) / 256;
  DKV_REQUIRE(blocks < (1L << 31), DKV_ESHAPE, "dkv_wire_pack: too many tokens");
  hipLaunchKernelGGL(wire_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, dkv::as_stream(stream), codes, low, scale,
                     rung, n, ladder, wire, out);
  return dkv::check_launch("dkv_wire_pack");
}

extern "C" int dkv_wire_unpack(const uint8_t* in, const int16_t* rung, int32_t n, dkv_ladder_t ladder,
                               dkv_wire_t wire, uint8_t* codes, uint16_t* low, uint16_t* scale, void* stream) {
  DKV_REQUIRE(n >= 0, DKV_ESHAPE, "dkv_wire_unpack: n < 0");
  int rc = dkv::check_ladder(ladder, "dkv_wire_unpack");
  if (rc) return rc;
  if ((rc = check_wire(wire, n, "dkv_wire_unpack"))) return rc;
  if (n == 0) return DKV_OK;
  DKV_REQUIRE(in && rung && codes && low && scale, DKV_EINVAL, "dkv_wire_unpack: null pointer");
  const long blocks = ((long)n * ladder.groups * 2 + 255) / 256;
  DKV_REQUIRE(blocks < (1L << 31), DKV_ESHAPE, "dkv_wire_unpack: too many tokens");
  hipLaunchKernelGGL(wire_unpack_kernel, dim3((unsigned)blocks), dim3(256), 0, dkv::as_stream(stream), in, rung, n,
                     ladder, wire, codes, low, scale);
  return dkv::check_launch("dkv_wire_unpack");
}

// ---------------------------------------------------------------------------
// K1: one thread per (token, group, half): 32 coefficients.
// ---------------------------------------------------------------------------
// Ladder streams: code * scale + low in fp32 (scripts/kvtc.py:78), then the
// output cast.  A rung outside the ladder decodes to zeros.
template <int DT>
DKV_DEVICE void unpack_ladder_half(const dkv_stream_t& s, int t, int g, int h, long base, void* __restrict__ out) {
  const int G = s.ladder.groups;
  const int r = s.pieces[t];
  const bool ok = r >= 0 && r < s.ladder.rungs;
  const int b = ok ? s.ladder.bits[(long)r * G + g] : 0;
  const uint8_t* seg = s.blob + s.tok_off[t] + (ok ? s.ladder.seg_off[(long)r * G + g] : 0);
  uint32_t cw[8], header;
  load_ladder_half(seg, b, h, cw, header);
  const float low = half_bits_to_float((uint16_t)(header & 0xffffu));
  const float scale = half_bits_to_float((uint16_t)(header >> 16));
#pragma unroll
  for (int w = 0; w < 8; ++w)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      store_from_float(out, base + 4 * w + i, DT, ladder_value((cw[w] >> (8 * i)) & 0xffu, low, scale));
}

template <int DT>
__global__ __launch_bounds__(256) void unpack_dequant_kernel(dkv_stream_t s, int t0, int nt, void* __restrict__ out) {
  const int G = dkv_groups(s);
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)nt * G * 2) return;
  const int h = (int)(id & 1);
  const long tg = id >> 1;
  const int tt = (int)(tg / G), g = (int)(tg % G);
  const int t = t0 + tt;
  if (s.format == DKV_FMT_LADDER) {
    unpack_ladder_half<DT>(s, t, g, h, (long)tt * (64L * G) + g * 64 + h * 32, out);
    return;
  }
  const int k = s.pieces[t];
  const int m = s.order.planes[(long)k * G + g];
  const uint8_t* seg = s.blob + s.tok_off[t] + s.order.seg_off[(long)k * G + g];
  uint32_t pl[8], header;
  load_segment(seg, m, h, pl, header);
  const float low = half_bits_to_float((uint16_t)(header & 0xffffu));
  const float span = half_bits_to_float((uint16_t)(header >> 16));
  const float inv_bins = __builtin_ldexpf(1.0f, -m);
  uint32_t cw[8];
  cw[0] = assemble_codes<0>(pl);
  cw[1] = assemble_codes<1>(pl);
  cw[2] = assemble_codes<2>(pl);
  cw[3] = assemble_codes<3>(pl);
  cw[4] = assemble_codes<4>(pl);
  cw[5] = assemble_codes<5>(pl);
  cw[6] = assemble_codes<6>(pl);
  cw[7] = assemble_codes<7>(pl);
  const long base = (long)tt * (64L * G) + g * 64 + h * 32;
  if (DT == DKV_F32) {
    float4* o = (float4*)((float*)out + base);
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      float4 v;
      v.x = dequant_exact(cw[w] & 0xffu, m, low, span, inv_bins);
      v.y = dequant_exact((cw[w] >> 8) & 0xffu, m, low, span, inv_bins);
      v.z = dequant_exact((cw[w] >> 16) & 0xffu, m, low, span, inv_bins);
      v.w = dequant_exact(cw[w] >> 24, m, low, span, inv_bins);
      o[w] = v;
    }
  } else {
#pragma unroll
    for (int w = 0; w < 8; ++w) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store_from_float(out, base + 4 * w + i, DT, dequant_exact((cw[w] >> (8 * i)) & 0xffu, m, low, span, inv_bins));
    }
  }
}

extern "C" int dkv_unpack_dequant(const dkv_stream_t* s, int32_t t0, int32_t nt, void* out, int32_t out_dtype,
                                  void* stream) {
  int rc = dkv::check_stream(s, "dkv_unpack_dequant");
  if (rc) return rc;
  DKV_REQUIRE(out, DKV_EINVAL, "dkv_unpack_dequant: out is null");
  DKV_REQUIRE(t0 >= 0 && nt >= 0, DKV_ESHAPE, "dkv_unpack_dequant: bad token range");
  DKV_REQUIRE(out_dtype == DKV_F32 || out_dtype == DKV_F16 || out_dtype == DKV_BF16, DKV_EINVAL,
              "dkv_unpack_dequant: bad dtype %d", out_dtype);
  if (nt == 0) return DKV_OK;
  const long threads = (long)nt * dkv::stream_groups(*s) * 2;
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  hipStream_t st = dkv::as_stream(stream);
  if (out_dtype == DKV_F32)
    hipLaunchKernelGGL(unpack_dequant_kernel<DKV_F32>, dim3(blocks), dim3(256), 0, st, *s, t0, nt, out);
  else if (out_dtype == DKV_F16)
    hipLaunchKernelGGL(unpack_dequant_kernel<DKV_F16>, dim3(blocks), dim3(256), 0, st, *s, t0, nt, out);
  else
    hipLaunchKernelGGL(unpack_dequant_kernel<DKV_BF16>, dim3(blocks), dim3(256), 0, st, *s, t0, nt, out);
  return dkv::check_launch("dkv_unpack_dequant");
}

// Reference dequantize on unpacked codes (progressive.py:47-55).
__global__ __launch_bounds__(256) void dequantize_codes_kernel(const uint8_t* __restrict__ codes,
                                                               const uint16_t* __restrict__ low,
                                                               const uint16_t* __restrict__ span,
                                                               const uint8_t* __restrict__ planes, int planes_rows,
                                                               int n, int G, float* __restrict__ out) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long)n * G * 64) return;
  const long tg = id >> 6;
  const int t = (int)(tg / G), g = (int)(tg % G);
  const int m = planes[(long)(planes_rows == 1 ? 0 : t) * G + g];
  const float lo = half_bits_to_float(low[tg]);
  const float sp = half_bits_to_float(span[tg]);
  out[id] = dequant_exact(codes[id], m, lo, sp, __builtin_ldexpf(1.0f, -m));
}

extern "C" int dkv_dequantize_codes(const uint8_t* codes, const uint16_t* low, const uint16_t* span,
                                    const uint8_t* planes, int32_t planes_rows, int32_t n, int32_t groups, float* out,
                                    void* stream) {
  DKV_REQUIRE(codes && low && span && planes && out, DKV_EINVAL, "dkv_dequantize_codes: null pointer");
  DKV_REQUIRE(n >= 0 && groups > 0 && (planes_rows == 1 || planes_rows == n), DKV_ESHAPE,
              "dkv_dequantize_codes: bad shape (n=%d groups=%d planes_rows=%d)", n, groups, planes_rows);
  if (n == 0) return DKV_OK;
  const long total = (long)n * groups * 64;
  hipLaunchKernelGGL(dequantize_codes_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     dkv::as_stream(stream), codes, low, span, planes, planes_rows, n, groups, out);
  return dkv::check_launch("dkv_dequantize_codes");
}

// ---------------------------------------------------------------------------
// Encoder: quantize8 (progressive.py:37-44) and the per-group squared error at
// 0..8 planes (progressive.py:152-158) in one pass over the coefficients.  One
// wave per (token, group), one lane per member: the group's min and max are
// wave reductions; low = f16(min), span = f16(max(max - low, 1e-8)),
// code = clamp(floor((x - low) / span * 256), 0, 255) with the division
// correctly rounded (a NaN from a zero fp16 span gives code 0); then every
// lane's squared error against the reference's dequantize at each plane count,
// summed over the wave.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quantize8_kernel(const float* __restrict__ coef, long ngroups,
                                                        uint8_t* __restrict__ codes, uint16_t* __restrict__ low,
                                                        uint16_t* __restrict__ span, float* __restrict__ errors) {
  const long tg = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (tg >= ngroups) return;
  const float x = coef[tg * 64 + lane];
  const float amin = -wave_max(-x), amax = wave_max(x);
  const half_t lo_h = (half_t)amin;
  const float lo = (float)lo_h;
  const half_t sp_h = (half_t)fmaxf(amax - lo, 1e-8f);
  const float sp = (float)sp_h;
  float q;
  {
#pragma clang fp contract(off)
    q = floorf(((x - lo) / sp) * 256.0f);
  }
  q = (q != q) ? 0.0f : fminf(fmaxf(q, 0.0f), 255.0f);
  const uint32_t code = (uint32_t)q;
  codes[tg * 64 + lane] = (uint8_t)code;
  if (lane == 0) {
    uint16_t lb, sb;
    __builtin_memcpy(&lb, &lo_h, 2);
    __builtin_memcpy(&sb, &sp_h, 2);
    low[tg] = lb;
    span[tg] = sb;
  }
  if (!errors) return;
  float mine = 0.0f;  // this lane ends up holding the error at (lane) planes, lane < 9
#pragma unroll
  for (int m = 0; m <= 8; ++m) {
    float d;
    {
#pragma clang fp contract(off)
      d = x - dequant_exact(code, m, lo, sp, __builtin_ldexpf(1.0f, -m));
      d = d * d;
    }
    const float e = wave_sum(d);
    mine = lane == m ? e : mine;
  }
  if (lane <= 8) errors[tg * 9 + lane] = mine;
}

extern "C" int dkv_quantize8(const float* coef, int32_t n, int32_t groups, uint8_t* codes, uint16_t* low,
                             uint16_t* span, float* errors, void* stream) {
  DKV_REQUIRE(coef && codes && low && span, DKV_EINVAL, "dkv_quantize8: null pointer");
  DKV_REQUIRE(n >= 0 && groups > 0, DKV_ESHAPE, "dkv_quantize8: bad shape (n=%d groups=%d)", n, groups);
  if (n == 0) return DKV_OK;
  const long ngroups = (long)n * groups;
  hipLaunchKernelGGL(quantize8_kernel, dim3((unsigned)((ngroups + 3) / 4)), dim3(256), 0, dkv::as_stream(stream),
                     coef, ngroups, codes, low, span, errors);
  return dkv::check_launch("dkv_quantize8");
}

// ---------------------------------------------------------------------------
// Centred token-matrix rows of the middle tokens, the encoders' input to the PCA projection
// (scripts/kvtc.py:137-140 to_matrix with :40-43 derotate and :50-53 token_matrix, then
// (matrix[start:end] - mean), :189 and scripts/progressive.py:147-148): row t - start, column
// f = (l * H + h) * D + d holds x - mean[f], x the cache element [l][0][h][t][d] as fp32 and, for
// keys, first de-rotated at position t: (k * cos - rotate_half(k) * sin) / (cos^2 + sin^2).  Every
// operation is rounded on its own, as the reference's separate tensor operations round them (no
// contraction), so the rows are bit-identical to that torch arithmetic.  One thread per 4
// consecutive columns of a row: consecutive threads write consecutive 16 bytes of the row.
// ---------------------------------------------------------------------------
template <int T>
DKV_DEVICE float4 load_elem4(const void* base, long idx) {
  if constexpr (T == DKV_F32) {
    return *(const float4*)((const float*)base + idx);
  } else {
    const uint2 w = *(const uint2*)((const uint16_t*)base + idx);
    const uint16_t e[4] = {(uint16_t)(w.x & 0xffffu), (uint16_t)(w.x >> 16), (uint16_t)(w.y & 0xffffu),
                           (uint16_t)(w.y >> 16)};
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = T == DKV_BF16 ? bf16_bits_to_float(e[i]) : half_bits_to_float(e[i]);
    return make_float4(v[0], v[1], v[2], v[3]);
  }
}

template <int T, bool ROTATE>
__global__ __launch_bounds__(256) void centered_rows_kernel(const uint64_t* __restrict__ layer_ptrs, int L, int H,
                                                            int tokens, int D, const float* __restrict__ cos,
                                                            const float* __restrict__ sin,
                                                            const float* __restrict__ mean, int start, long quads,
                                                            float* __restrict__ out) {
  const long q = (long)blockIdx.x * 256 + threadIdx.x;
  if (q >= quads) return;
  const int D4 = D / 4;
  const int d4 = (int)(q % D4);
  const long r = q / D4;  // (t, l, h) with h fastest
  const int h = (int)(r % H), l = (int)((r / H) % L);
  const int t = start + (int)(r / ((long)H * L));
  const int d = 4 * d4;
  const void* base = (const void*)layer_ptrs[l];
  const long row = (long)h * tokens + t;  // the cache element [l][0][h][t][.]
  const float4 x = load_elem4<T>(base, row * D + d);
  const long f = ((long)l * H + h) * D + d;
  const float4 mu = *(const float4*)(mean + f);
  float v[4] = {x.x, x.y, x.z, x.w};
  if constexpr (ROTATE) {
    const int half = D / 2;
    // rotate_half: -k[d + D/2] for d < D/2, k[d - D/2] above
    const bool lower = d < half;
    const float4 p = load_elem4<T>(base, row * D + (lower ? d + half : d - half));
    const float4 c4 = *(const float4*)(cos + (long)t * D + d);
    const float4 s4 = *(const float4*)(sin + (long)t * D + d);
    const float pv[4] = {p.x, p.y, p.z, p.w}, cv[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)
      const float rh = lower ? -pv[i] : pv[i];
      const float num = v[i] * cv[i] - rh * sv[i];
      const float den = cv[i] * cv[i] + sv[i] * sv[i];
      v[i] = num / den;
    }
  }
  float4 o;
  {
#pragma clang fp contract(off)
    o = make_float4(v[0] - mu.x, v[1] - mu.y, v[2] - mu.z, v[3] - mu.w);
  }
  *(float4*)(out + (long)(t - start) * ((long)L * H * D) + f) = o;
}

extern "C" int dkv_centered_rows(const uint64_t* layer_ptrs, int32_t dtype, int32_t layers, int32_t heads,
                                 int32_t tokens, int32_t head_dim, const float* cos, const float* sin,
                                 const float* mean, int32_t start, int32_t end, float* out, void* stream) {
  DKV_REQUIRE(layer_ptrs && mean && out, DKV_EINVAL, "dkv_centered_rows: null pointer");
  DKV_REQUIRE((cos == nullptr) == (sin == nullptr), DKV_EINVAL, "dkv_centered_rows: cos and sin go together");
  DKV_REQUIRE(dtype == DKV_F32 || dtype == DKV_F16 || dtype == DKV_BF16, DKV_EINVAL,
              "dkv_centered_rows: dtype %d not supported", dtype);
  DKV_REQUIRE(layers > 0 && heads > 0 && tokens >= 0 && head_dim > 0 && head_dim % 8 == 0, DKV_ESHAPE,
              "dkv_centered_rows: bad shape (layers=%d heads=%d tokens=%d head_dim=%d)", layers, heads, tokens,
              head_dim);
  DKV_REQUIRE(0 <= start && start <= end && end <= tokens, DKV_ESHAPE,
              "dkv_centered_rows: rows %d..%d outside 0..%d", start, end, tokens);
  const long quads = (long)(end - start) * layers * heads * (head_dim / 4);
  if (quads == 0) return DKV_OK;
  const dim3 grid((unsigned)((quads + 255) / 256));
  hipStream_t st = dkv::as_stream(stream);
#define DKV_CENTERED(T_, R_)                                                                                    \
  hipLaunchKernelGGL((centered_rows_kernel<T_, R_>), grid, dim3(256), 0, st, layer_ptrs, layers, heads, tokens, \
                     head_dim, cos, sin, mean, start, quads, out)
  const bool rot = cos != nullptr;
  if (dtype == DKV_F16) {
    if (rot) DKV_CENTERED(DKV_F16, true); else DKV_CENTERED(DKV_F16, false);
  } else if (dtype == DKV_BF16) {
    if (rot) DKV_CENTERED(DKV_BF16, true); else DKV_CENTERED(DKV_BF16, false);
  } else {
    if (rot) DKV_CENTERED(DKV_F32, true); else DKV_CENTERED(DKV_F32, false);
  }
#undef DKV_CENTERED
  return dkv::check_launch("dkv_centered_rows");
}

// ---------------------------------------------------------------------------
// K4c: merge hot + cold segments of selected tokens into full blobs.
// One workgroup per selected token; one thread per group.
// ---------------------------------------------------------------------------
// Merges token t's hot and cold segments into the full blob at refined + r * full_bytes and points the
// stream at it (one workgroup; one thread per group).
DKV_DEVICE void gather_token(const dkv_stream_t& s, const uint8_t* __restrict__ cold,
                             const int64_t* __restrict__ cold_tok_off, int t, int r, uint8_t* __restrict__ refined,
                             int64_t refined_base_off, int64_t* tok_off, int16_t* pieces) {
  const int G = s.order.groups, K = s.order.pieces;
  const int k = pieces[t];
  const int64_t off = tok_off[t];
  const int full_bytes = s.order.prefix_bytes[K];
  uint8_t* dst_tok = refined + (long)r * full_bytes;
  // One group per thread.  The full segment is the header and m_full plane words (at most 17
  // 32-bit words); word i comes from the hot segment (header and planes below m_hot) or the cold
  // one (the header when m_hot = 0, then planes m_hot..).  Every word's source is selected first
  // and all loads go out together (words past the segment re-read the header and are not stored).
  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    const int m_hot = s.order.planes[(long)k * G + g];
    const int m_full = s.order.planes[(long)K * G + g];
    if (m_full == 0) continue;
    uint32_t* dst = (uint32_t*)(dst_tok + s.order.seg_off[(long)K * G + g]);
    const uint32_t* hseg = (const uint32_t*)(s.blob + off + s.order.seg_off[(long)k * G + g]);
    const uint32_t* cseg = (const uint32_t*)(cold + cold_tok_off[t] + s.order.cold_off[(long)k * G + g]);
    const uint32_t* head = m_hot > 0 ? hseg : cseg;
    const uint32_t* cplanes = m_hot > 0 ? cseg : cseg + 1;  // the cold part's plane words
    const int words = 1 + 2 * m_full;
    uint32_t v[17];
    v[0] = head[0];
#pragma unroll
    for (int i = 1; i < 17; ++i) {
      const int p = (i - 1) >> 1, j = (i - 1) & 1;
      const uint32_t* src = i >= words ? head : p < m_hot ? hseg + 1 + 2 * p + j : cplanes + 2 * (p - m_hot) + j;
      v[i] = *src;
    }
#pragma unroll
    for (int i = 0; i < 17; ++i)
      if (i < words) dst[i] = v[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    tok_off[t] = refined_base_off + (int64_t)r * full_bytes;
    pieces[t] = (int16_t)K;
  }
}


__global__ __launch_bounds__(64) void gather_cold_kernel(dkv_stream_t s, const uint8_t* __restrict__ cold,
                                                         const int64_t* __restrict__ cold_tok_off,
                                                         const int32_t* __restrict__ idx, uint8_t* __restrict__ refined,
                                                         int64_t refined_base_off, int64_t* tok_off,
                                                         int16_t* pieces) {
  gather_token(s, cold, cold_tok_off, idx[blockIdx.x], blockIdx.x, refined, refined_base_off, tok_off, pieces);
}

// ---------------------------------------------------------------------------
// K4c over any token list, without a host round trip.  refine_prepare_kernel:
// one thread per entry r of rows; in-range entries add the reference's cold
// bytes (full size - hot prefix of the token's current pieces,
// progressive.py:232) to fetched[0] and claim the token in owner[t] with the
// key (version << 32) | (2^31 - 1 - r): the largest key of this version is the
// token's first entry, and older versions' keys are smaller, so owner never
// needs clearing.  An entry outside 0..n-1 sets fetched[1].  The gather then
// runs one workgroup per entry and merges a token only from its first entry,
// and none at all if fetched[1] is set.  Integer sums: the result does not
// depend on the order in which entries are added.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void refine_prepare_kernel(const int32_t* __restrict__ rows, int k, int n,
                                                             const int16_t* __restrict__ pieces,
                                                             const int32_t* __restrict__ prefix_bytes, int K,
                                                             int64_t* owner, int64_t version, int64_t* fetched) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= k) return;
  const int t = rows[r];
  if (t < 0 || t >= n) {
    atomicOr((unsigned long long*)&fetched[1], 1ull);
    return;
  }
  const int64_t bytes = (int64_t)prefix_bytes[K] - prefix_bytes[pieces[t]];
  atomicAdd((unsigned long long*)&fetched[0], (unsigned long long)bytes);
  atomicMax((unsigned long long*)&owner[t], (unsigned long long)((version << 32) | (int64_t)(0x7fffffff - r)));
}

__global__ __launch_bounds__(64) void gather_owned_kernel(dkv_stream_t s, const uint8_t* __restrict__ cold,
                                                          const int64_t* __restrict__ cold_tok_off,
                                                          const int32_t* __restrict__ rows, int n,
                                                          uint8_t* __restrict__ refined, int64_t refined_base_off,
                                                          int64_t* tok_off, int16_t* pieces,
                                                          const int64_t* __restrict__ owner, int64_t version,
                                                          const int64_t* __restrict__ fetched) {
  const int r = blockIdx.x;
  const int t = rows[r];
  // uniform per workgroup: a bad list changes nothing; a repeated token is merged from its first entry
  if (fetched[1] != 0 || t < 0 || t >= n) return;
  if (owner[t] != ((version << 32) | (int64_t)(0x7fffffff - r))) return;
  gather_token(s, cold, cold_tok_off, t, r, refined, refined_base_off, tok_off, pieces);
}

extern "C" int dkv_gather_cold(const dkv_stream_t* s, const uint8_t* cold, const int64_t* cold_tok_off,
                               const int32_t* idx, int32_t k, uint8_t* refined, int64_t refined_base_off,
                               int64_t* tok_off, int16_t* pieces, void* stream) {
  int rc = dkv::check_stream(s, "dkv_gather_cold");
  if (rc) return rc;
  DKV_REQUIRE(s->format == DKV_FMT_PLANES, DKV_EINVAL, "dkv_gather_cold: only bit-plane streams have a cold tier");
  DKV_REQUIRE(cold && cold_tok_off && idx && refined && tok_off && pieces && s->order.cold_off, DKV_EINVAL,
              "dkv_gather_cold: null pointer");
  DKV_REQUIRE(k >= 0 && refined_base_off >= 0, DKV_ESHAPE, "dkv_gather_cold: bad k / offset");
  if (k == 0) return DKV_OK;
  dkv_stream_t view = *s;
  hipLaunchKernelGGL(gather_cold_kernel, dim3(k), dim3(64), 0, dkv::as_stream(stream), view, cold, cold_tok_off, idx,
                     refined, refined_base_off, tok_off, pieces);
  return dkv::check_launch("dkv_gather_cold");
}

extern "C" int dkv_refine_rows(const dkv_stream_t* s, int32_t n, const uint8_t* cold, const int64_t* cold_tok_off,
                               const int32_t* rows, int32_t k, uint8_t* refined, int64_t refined_base_off,
                               int64_t* tok_off, int16_t* pieces, int64_t* owner, int32_t version, int64_t* fetched,
                               void* stream) {
  int rc = dkv::check_stream(s, "dkv_refine_rows");
  if (rc) return rc;
  DKV_REQUIRE(s->format == DKV_FMT_PLANES, DKV_EINVAL, "dkv_refine_rows: only bit-plane streams have a cold tier");
  DKV_REQUIRE(cold && cold_tok_off && rows && refined && tok_off && pieces && owner && fetched && s->order.cold_off,
              DKV_EINVAL, "dkv_refine_rows: null pointer");
  DKV_REQUIRE(n >= 0 && k >= 0 && refined_base_off >= 0 && version > 0, DKV_ESHAPE,
              "dkv_refine_rows: bad n / k / offset / version");
  if (k == 0) return DKV_OK;
  const hipStream_t st = dkv::as_stream(stream);
  hipLaunchKernelGGL(refine_prepare_kernel, dim3((unsigned)((k + 255) / 256)), dim3(256), 0, st, rows, k, n,
                     (const int16_t*)pieces, s->order.prefix_bytes, s->order.pieces, owner, (int64_t)version, fetched);
  rc = dkv::check_launch("dkv_refine_rows");
  if (rc) return rc;
  dkv_stream_t view = *s;
  hipLaunchKernelGGL(gather_owned_kernel, dim3(k), dim3(64), 0, st, view, cold, cold_tok_off, rows, n, refined,
                     refined_base_off, tok_off, pieces, (const int64_t*)owner, (int64_t)version, (const int64_t*)fetched);
  return dkv::check_launch("dkv_refine_rows");
}

// ---------------------------------------------------------------------------
// Basis layouts.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void key_basis_kernel(const float* __restrict__ basis, int L, int H, int D, int R,
                                                        uint16_t* __restrict__ out) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)L * H * D * R;
  if (id >= total) return;
  // out index = (((l*G + g)*H + h)*D + dd)*64 + kk
  const int G = R / 64;
  const int kk = (int)(id & 63);
  long rest = id >> 6;
  const int dd = (int)(rest % D);
  rest /= D;
  const int h = (int)(rest % H);
  rest /= H;
  const int g = (int)(rest % G);
  const int l = (int)(rest / G);
  const float v = basis[((long)(l * H + h) * D + dd) * R + g * 64 + kk];
  half_t hv = (half_t)v;
  uint16_t bits;
  __builtin_memcpy(&bits, &hv, 2);
  out[id] = bits;
}

__global__ __launch_bounds__(256) void value_basis_kernel(const float* __restrict__ basis, int L, int H, int D, int R,
                                                          uint16_t* __restrict__ out) {
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)L * H * D * R;
  if (id >= total) return;
  // out index = ((l*H + h)*R + k)*D + dd
  const int dd = (int)(id % D);
  long rest = id / D;
  const int k = (int)(rest % R);
  const long lh = rest / R;
  const float v = basis[(lh * D + dd) * R + k];
  half_t hv = (half_t)v;
  uint16_t bits;
  __builtin_memcpy(&bits, &hv, 2);
  out[id] = bits;
}

static int check_basis_args(const float* basis, int L, int H, int D, int R, const uint16_t* out, const char* what) {
  DKV_REQUIRE(basis && out, DKV_EINVAL, "%s: null pointer", what);
  DKV_REQUIRE(L > 0 && H > 0 && D > 0 && R > 0 && R % 64 == 0, DKV_ESHAPE, "%s: bad shape L=%d H=%d D=%d R=%d", what,
              L, H, D, R);
  return DKV_OK;
}

extern "C" int dkv_prepare_key_basis(const float* basis, int32_t layers, int32_t kv_heads, int32_t head_dim,
                                     int32_t rank, uint16_t* out, void* stream) {
  int rc = check_basis_args(basis, layers, kv_heads, head_dim, rank, out, "dkv_prepare_key_basis");
  if (rc) return rc;
  const long total = (long)layers * kv_heads * head_dim * rank;
  hipLaunchKernelGGL(key_basis_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, dkv::as_stream(stream),
                     basis, layers, kv_heads, head_dim, rank, out);
  return dkv::check_launch("dkv_prepare_key_basis");
}

extern "C" int dkv_prepare_value_basis(const float* basis, int32_t layers, int32_t kv_heads, int32_t head_dim,
                                       int32_t rank, uint16_t* out, void* stream) {
  int rc = check_basis_args(basis, layers, kv_heads, head_dim, rank, out, "dkv_prepare_value_basis");
  if (rc) return rc;
  const long total = (long)layers * kv_heads * head_dim * rank;
  hipLaunchKernelGGL(value_basis_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, dkv::as_stream(stream),
                     basis, layers, kv_heads, head_dim, rank, out);
  return dkv::check_launch("dkv_prepare_value_basis");
}
