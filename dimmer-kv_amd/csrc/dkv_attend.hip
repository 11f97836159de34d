// One layer of attention directly over the packed bit-plane codes.
//
// Replaces scripts/compressed_attention.py:105-137 (CompressedContext._keys /
// attend) of SrikanthBalaaji/Dimmer-KV, applied to progressive codes
// (scripts/progressive.py:47-55, 196-201):
//
//   K1  decode_keys / decode_values (once per decode step, read by every
//                      layer): the packed hot tier -> key coefficients as fp16
//                      in the 32x32x16 MFMA operand order, and value codes as
//                      8-bit codes blocked by 16 slots with one (scale,
//                      offset) pair per (token, group).
//   K2  keys_scores  : per (256-token tile, head group) - multiply the decoded
//                      key coefficients (one 16-byte operand load per lane)
//                      by the layer's key-basis slice (double-buffered in LDS)
//                      on MFMA (32x32x16 f16, fp32 accumulate, starting at
//                      the key mean), apply RoPE at the token positions and
//                      score against the GQA query rows in registers, write
//                      fp16 probabilities relative to the tile maximum and
//                      per-tile (max, sum exp) statistics.  The rebuilt keys
//                      never reach memory.  Decodes whose (tile, head group)
//                      workgroups would leave CUs idle run one workgroup per
//                      (tile, KV head) instead (keys_scores_head), or per
//                      (half tile, KV head) for the shortest contexts.
//   K3a value_weights: per (1024-token split, 64-component group, 32 rows):
//                      p @ value codes on MFMA plus sum(p * offset) ->
//                      coefficient-space partial sums.
//   K3b basis_apply  : sum the partials over the splits and multiply once by
//                      the value basis of the KV head (per 128-component
//                      chunk and 64-dimension slice); beside them, four
//                      one-wave workgroups per output row compute the exact
//                      tail (sinks, recent window, new tokens), a share of
//                      its tokens each: scores, their maximum and
//                      exponential sum, and the weighted values.
//   K3c finish       : per output row, merge the tiles' softmax statistics
//                      (Mc, Lc) with the exact tail's shares (Me, Le, ve) in one
//                      softmax: out = (ec (sum of chunk partials + Lc mean_v)
//                      + ee ve) / (ec Lc + ee Le), ec and ee taking Mc and Me
//                      to the common maximum.
#include <math.h>

#include <mutex>
#include <type_traits>
#include <utility>

#include "dkv_device.h"
#include "dkv_host.h"

namespace {

constexpr int kTileTok = 256;    // tokens per K2 workgroup
constexpr int kK2Threads = 512;  // 8 waves: 4 token quarters x 2 row halves
constexpr int kStride = 72;      // LDS row stride in halves for [row][64] tiles (64 + 8 pad)
constexpr int kSplitTok = 1024;  // tokens per K3a split (512 when 1024-token splits leave CUs idle)
constexpr int kChunk = 128;      // components per K3b workgroup

constexpr int kMaxExact = 1024;
constexpr int kRowThreads = 256;  // threads of a row workgroup (the exact tail in K3b, the merge in K3c)

struct RowMergeArgs {
  const int32_t* cu_seqlens;
  const int32_t* cu_exact;
  const float* tile_max;
  const float* tile_sum;
  const float* mean_v;
  const void* key_exact;    // [Hkv][E_total][D] in the exact tail's type (row_exact's XT)
  const void* value_exact;
  const float* mask;
  const void* query;
  const float* out_part;  // [nchunks][batch * R_total][D] value-basis chunk partials (K3b)
  float* ex;              // [batch * R_total][kExactParts][D + 2] per row and share: Me, Le, then ve[D] (row_exact)
  void* out;              // [batch][q_len][Hq][D], out_dtype
  float scaling;
  // nstats: softmax-statistics entries per row (ntiles, or 2 * ntiles for 128-token entries)
  int batch, n_total, layer, Hkv, Hq, q_len, D, R_total, E_total, query_dtype, nstats, nchunks, out_dtype;
  int e0_single, e_single;  // with one sequence: its first exact token and exact-token count
};

struct K2Args {
  const uint16_t* coef;  // decoded key coefficients, MFMA fragment order over slots
  const int32_t* cu_seqlens;
  const int32_t* positions;
  const uint16_t* key_basis;
  const float* mean_k;
  const float* rope_cos;
  const float* rope_sin;
  const void* query;
  uint16_t* probs;  // fp16 exp(score - tile max) (decoding) or exp(score - quarter max) (question scoring)
  float* tile_max;
  float* tile_sum;
  float scaling;
  int batch, layer, Hkv, Hq, q_len, G, n_total, n_slots, ntiles, total_wg, per_xcd, query_dtype;
  int rope_rows;  // rows of the RoPE tables: positions are clamped to 0 .. rope_rows - 1
  // question scoring: (max, sum exp) of every row over each 64-token quarter of a tile, [R][ntiles * 4]
  float* sub_max;
  float* sub_sum;
  int nstats;  // softmax-statistics entries per row: ntiles, or 2 * ntiles with 128-token entries
};

DKV_DEVICE uint16_t f16_bits(float v) {
  half_t h = (half_t)v;
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// f16_bits(lo) | f16_bits(hi) << 16 as one v_cvt_pk_f16_f32 (both rounded to nearest even).
DKV_DEVICE uint32_t pack_f16x2(float lo, float hi) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const half2_t v = {(half_t)lo, (half_t)hi};
  return __builtin_bit_cast(uint32_t, v);
}

DKV_DEVICE half8 lds_half8(const half_t* p) { return *(const half8*)p; }

// The query type as a compile-time tag: a kernel section instantiated per type issues its query
// loads back to back, where a type switch around each load would make every load wait for the last.
template <int T>
struct QueryType {
  static constexpr int value = T;
};

// 8 consecutive query elements (idx a multiple of 8) of type T as fp16.
template <int T>
DKV_DEVICE half8 load_query8_t(const void* q, long idx) {
  half8 r;
  if constexpr (T == DKV_F16) {
    r = *(const half8*)((const half_t*)q + idx);
  } else if constexpr (T == DKV_BF16) {
    const uint4 v = *(const uint4*)((const uint16_t*)q + idx);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[2 * i] = (half_t)__uint_as_float(w[i] << 16);
      r[2 * i + 1] = (half_t)__uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const float4 x = *(const float4*)((const float*)q + idx);
    const float4 y = *(const float4*)((const float*)q + idx + 4);
    r[0] = (half_t)x.x; r[1] = (half_t)x.y; r[2] = (half_t)x.z; r[3] = (half_t)x.w;
    r[4] = (half_t)y.x; r[5] = (half_t)y.y; r[6] = (half_t)y.z; r[7] = (half_t)y.w;
  }
  return r;
}

// One query element as the aligned 32-bit word that holds it: one unconditional load whatever the
// type (a 16-bit tensor has an even element count, so the word never passes its end), converted
// once the value is needed.
DKV_DEVICE uint32_t load_query_word(const void* q, long idx, int dtype) {
  return *(const uint32_t*)((const char*)q + (dtype == DKV_F32 ? idx * 4 : ((idx * 2) & ~3L)));
}

DKV_DEVICE float query_word_value(uint32_t w, long idx, int dtype) {
  const uint16_t h = (uint16_t)(w >> ((idx & 1) * 16));
  return dtype == DKV_F32 ? __uint_as_float(w) : dtype == DKV_BF16 ? bf16_bits_to_float(h) : half_bits_to_float(h);
}

// A query fragment as it travels from memory to the MFMA: fp16 and bf16 fragments stay raw
// 16-byte words until they are used, so their loads can be waited for late; fp32 fragments (two
// 16-byte loads) are converted when loaded.
template <int T>
struct QueryFrag {
  using type = uint4;
};
template <>
struct QueryFrag<DKV_F32> {
  using type = half8;
};

template <int T>
DKV_DEVICE typename QueryFrag<T>::type load_query_frag(const void* q, long idx) {
  if constexpr (T == DKV_F32)
    return load_query8_t<DKV_F32>(q, idx);
  else
    return *(const uint4*)((const uint16_t*)q + idx);
}

// 8 query elements as loaded, before conversion (two 16-byte words for fp32), so that a batch of
// loads goes out before the first conversion waits for its data.
template <int T>
struct RawQuery8 {
  uint4 w;
};
template <>
struct RawQuery8<DKV_F32> {
  float4 x, y;
};

template <int T>
DKV_DEVICE RawQuery8<T> load_raw_query8(const void* q, long idx) {
  RawQuery8<T> r;
  if constexpr (T == DKV_F32) {
    r.x = *(const float4*)((const float*)q + idx);
    r.y = *(const float4*)((const float*)q + idx + 4);
  } else {
    r.w = *(const uint4*)((const uint16_t*)q + idx);
  }
  return r;
}

template <int T>
DKV_DEVICE half8 query_frag_half(const typename QueryFrag<T>::type& f);

template <int T>
DKV_DEVICE half8 raw_query8_half(const RawQuery8<T>& r) {
  if constexpr (T == DKV_F32) {
    half8 h;
    h[0] = (half_t)r.x.x; h[1] = (half_t)r.x.y; h[2] = (half_t)r.x.z; h[3] = (half_t)r.x.w;
    h[4] = (half_t)r.y.x; h[5] = (half_t)r.y.y; h[6] = (half_t)r.y.z; h[7] = (half_t)r.y.w;
    return h;
  } else {
    return query_frag_half<T>(r.w);
  }
}

template <int T>
DKV_DEVICE half8 query_frag_half(const typename QueryFrag<T>::type& f) {
  if constexpr (T == DKV_F32) {
    return f;
  } else if constexpr (T == DKV_F16) {
    half8 r;
    __builtin_memcpy(&r, &f, 16);
    return r;
  } else {
    half8 r;
    const uint32_t w[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[2 * i] = (half_t)__uint_as_float(w[i] << 16);
      r[2 * i + 1] = (half_t)__uint_as_float(w[i] & 0xffff0000u);
    }
    return r;
  }
}

// ---------------------------------------------------------------------------
// Token slots.  Every sequence's compressed tokens are cut into tiles of 256
// (the K2 tile; the last tile of a sequence may be partial) and tile i owns
// slots 256*i .. 256*i+255 of the decoded buffers, so every tile starts at an
// aligned slot and its unused slots are padding that decodes to zero.  The
// buffers hold n_slots = 256 * ntiles + kSplitTok slots: a K3a split (4 tiles)
// starting at any tile stays inside them.
// ---------------------------------------------------------------------------
struct DecodeArgs {
  dkv_stream_t s;
  const int32_t* cu_seqlens;
  uint16_t* coef;  // keys: fp16 in MFMA fragment order (see decode_keys_block)
  int batch, n_total, ntiles, n_slots, G, plane_cap;
};

constexpr int kDecodeSlots = 256;      // slots per decode workgroup: one thread per (slot, group)
constexpr int kMaxTableRows = 4096;    // rows of a stream table one decode workgroup stages in LDS

// Block -> (slot block, group) with the group fastest and consecutive ids on
// one XCD, so the blocks reading the same tokens' blobs share that XCD's L2.
DKV_DEVICE int2 decode_block(int G, int nblocks, int id) {
  const int per_xcd = (nblocks + 7) / 8;
  const int lin = (id & 7) * per_xcd + (id >> 3);
  return make_int2(lin / G, lin % G);  // (slot block, group); slot block may be out of range
}

// Rows of a stream's per-token table: piece counts 0..K of the plane format, rungs of the ladder.
DKV_DEVICE int table_rows(const dkv_stream_t& s) {
  return s.format == DKV_FMT_LADDER ? s.ladder.rungs : s.order.pieces + 1;
}

// Group g's column of the stream table staged in LDS as (planes or bits, segment offset) per
// row, so that a thread's segment address follows from its token's row without a dependent
// global load.  The caller synchronises before reading it.
DKV_DEVICE void stage_table_column(const dkv_stream_t& s, int G, int g, int2* tab) {
  const bool ladder = s.format == DKV_FMT_LADDER;
  const uint8_t* cnt = ladder ? s.ladder.bits : s.order.planes;
  const int32_t* off = ladder ? s.ladder.seg_off : s.order.seg_off;
  const int rows = table_rows(s);
  for (int r = threadIdx.x; r < rows; r += blockDim.x)
    tab[r] = make_int2(cnt[(long)r * G + g], off[(long)r * G + g]);
}

// The (token, group) segment of `slot`'s token, whole: header and code words, with its plane count
// (plane format, capped at plane_cap) or bit width (ladder).  Padding slots and rows outside the
// table give an empty segment.  tok_row / tok_off are the token's table row and blob offset,
// loaded by the caller beside the table column.
struct SegmentWords {
  uint32_t header;
  uint32_t w[16];
  int m;  // planes (plane format) or bits (ladder); 0 for an empty segment
};

DKV_DEVICE SegmentWords load_token_segment(const dkv_stream_t& s, const int2* tab, int t, int row, long tok_off,
                                           int plane_cap) {
  SegmentWords sw;
  const bool ok = t >= 0 && row >= 0 && row < table_rows(s);
  const int2 e = ok ? tab[row] : make_int2(0, 0);
  const int m = s.format == DKV_FMT_LADDER ? e.x : min(e.x, plane_cap);
  sw.m = m;
  if (s.format == DKV_FMT_LADDER)
    load_ladder_segment(s.blob + tok_off + e.y, m, sw.header, sw.w);
  else
    load_segment_words(s.blob + tok_off + e.y, 2 * m, sw.header, sw.w);
  return sw;
}

// Token held by `slot`, or -1 for a padding slot.
DKV_DEVICE int slot_token(const DecodeArgs& a, int slot) {
  const int tile = slot / kTileTok;
  if (tile >= a.ntiles) return -1;
  const int2 bt = find_tile(a.cu_seqlens, a.batch, a.n_total, kTileTok, tile);
  const int2 sr = seq_range(a.cu_seqlens, a.batch, a.n_total, bt.x);
  const int tok0 = sr.x + bt.y * kTileTok;
  const int n = slot - tile * kTileTok;
  return n < sr.y - tok0 ? tok0 + n : -1;
}

// The value side's per-step buffers are blocked by 16 slots so that a wave's
// MFMA operand loads are whole cache lines:
//   value codes    u8   [G][n_slots/16][64 components][16 slots]
//   probabilities  fp16 [n_slots/16][R_total rows][16 slots]
DKV_DEVICE long vcode_index(int g, int c, long slot, int n_slots) {
  return (((long)g * (n_slots >> 4) + (slot >> 4)) * 64 + c) * 16 + (slot & 15);
}

DKV_DEVICE long prob_index(long row, long slot, int R_total) {
  return ((slot >> 4) * R_total + row) * 16 + (slot & 15);
}

// Question scoring's per-quarter statistics, [R/8][nsub][8]: eight consecutive rows sit together for
// each 64-token quarter t, so a wave's 32 rows store four 32-byte pieces and the row-statistics
// kernel reads its eight rows' quarters as one contiguous run.
DKV_DEVICE long sub_index(long row, int t, int nsub) { return ((row >> 3) * nsub + t) * 8 + (row & 7); }


// ---------------------------------------------------------------------------
// K1 (fp16 operand form): decode the hot key codes of every token into the
// exact register image of a 32x32x16 MFMA operand: for 64-component group g,
// 32-slot block j and 16-component step ks, lane l (0..63) holds components
// ks*16 + (l/32)*8 .. +8 of slot 32j + l%32, so K2 loads each operand with one
// coalesced 16-byte load per lane.  Values are the affine dequantization of
// the codes truncated to min(m, plane_cap) planes.  One thread per (slot,
// group): two load rounds (the token's row and blob offset beside the
// group's table column, then the segment in 16-byte pieces) and eight
// 16-byte stores.  The decoded keys depend on the stream only, so one decode
// serves every layer.
// ---------------------------------------------------------------------------
DKV_DEVICE void decode_keys_block(const DecodeArgs& a, int2* tab, int id) {
  const int nsb = a.n_slots / kDecodeSlots;
  const int2 bg = decode_block(a.G, nsb * a.G, id);
  const int sb = bg.x, g = bg.y;
  if (sb >= nsb) return;  // the whole block
  const int slot = sb * kDecodeSlots + threadIdx.x;
  const int t = slot_token(a, slot);
  const int row = t >= 0 ? a.s.pieces[t] : 0;
  const long toff = t >= 0 ? a.s.tok_off[t] : 0;
  stage_table_column(a.s, a.G, g, tab);
  __syncthreads();
  const SegmentWords sw = load_token_segment(a.s, tab, t, row, toff, a.plane_cap);
  uint32_t vals[2][16];  // half h: components 32h .. 32h+31 as packed fp16 pairs
  if (a.s.format == DKV_FMT_LADDER) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t cw[8];
      ladder_segment_half(sw.w, sw.m, h, cw);
      ladder_half_f16(cw, sw.header, vals[h]);
    }
  } else {
    const AffineDq dq = affine_from_header(sw.header, sw.m);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t pl[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) pl[q] = sw.w[2 * q + h];
      unpack_half_f16(pl, dq, vals[h]);
    }
  }
  // components 8c .. 8c+7 (c = 0..7) go to step ks = c/2, lane half c%2 of the slot's 32-slot block
  const long blk = (long)g * (a.n_slots / 32) + slot / 32;
  const int l32 = slot % 32;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t* v = &vals[c / 4][4 * (c % 4)];
    uint4* dst = (uint4*)(a.coef + ((blk * 4 + c / 2) * 64 + (c % 2) * 32 + l32) * 8);
    *dst = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// ---------------------------------------------------------------------------
// K2 epilogue for few query rows per KV head (decode: RH = (Hq/Hkv) * q_len
// <= kSmallRows).  The keys never leave registers: the tile's RoPE rows are
// staged in LDS (coalesced), each lane rotates the dimension pairs it holds
// (d and d + D/2 sit in the same lane) and dots them with the query rows in
// fp32; the two lanes holding the two halves of a token's dimensions combine
// with one shuffle.  Scores and per-tile softmax statistics are written as in
// the MFMA epilogue.
// ---------------------------------------------------------------------------
constexpr int kSmallRows = 4;

// Stage the RoPE rows (cos and sin, [256][D/2 + 4] floats each) of the tile's tokens in LDS, with
// coalesced loads: positions from pos_s, the loads of a batch issued together, rows past the tile's
// tokens replaced by (1, 0) afterwards.  Ends with a barrier.
template <int D>
DKV_DEVICE void stage_rope_rows(const K2Args& a, float* cs, float* sn, const int* pos_s, int count) {
  constexpr int HALF_D = D / 2;
  constexpr int CSTR = HALF_D + 4;
  constexpr int V4_PER_ROW = HALF_D / 4;
  constexpr int STAGE_ITERS = kTileTok * V4_PER_ROW / kK2Threads;  // 8 (D = 128) or 4 (D = 64)
  constexpr int STAGE_BATCH = 4;  // (one round of 8 measured slower: the main loop's registers)
  const int tid = threadIdx.x;
#pragma unroll
  for (int i0 = 0; i0 < STAGE_ITERS; i0 += STAGE_BATCH) {
    long pos[STAGE_BATCH];
#pragma unroll
    for (int i = 0; i < STAGE_BATCH; ++i) pos[i] = pos_s[(tid + (i0 + i) * kK2Threads) / V4_PER_ROW];
    float4 cv[STAGE_BATCH], sv[STAGE_BATCH];
#pragma unroll
    for (int i = 0; i < STAGE_BATCH; ++i) {
      const int c = (tid + (i0 + i) * kK2Threads) % V4_PER_ROW;
      cv[i] = *(const float4*)(a.rope_cos + pos[i] * HALF_D + 4 * c);
      sv[i] = *(const float4*)(a.rope_sin + pos[i] * HALF_D + 4 * c);
    }
#pragma unroll
    for (int i = 0; i < STAGE_BATCH; ++i) {
      const int e = tid + (i0 + i) * kK2Threads;
      const int n = e / V4_PER_ROW, c = e % V4_PER_ROW;
      const bool ok = n < count;
      *(float4*)(cs + n * CSTR + 4 * c) = ok ? cv[i] : make_float4(1.f, 1.f, 1.f, 1.f);
      *(float4*)(sn + n * CSTR + 4 * c) = ok ? sv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __syncthreads();
}

// One RoPE table (cos or sin, [rope_rows][D/2] floats) of the tile's 256 tokens straight into LDS
// (global_load_lds: no registers), unpadded and swizzled: token n's 16-byte piece c sits at piece
// n * NC + (c ^ (n % NC)) of dst (NC = D/8 pieces per token), which keeps the epilogue's reads of a
// piece across 32 consecutive tokens on distinct banks.  Each wave instruction fills 64 consecutive
// pieces (1 KB); lane l takes piece S0 + l and loads whichever source piece the swizzle puts
// there.  Positions come from pos_s (past the tile's tokens, its last token's, so every row is a
// real table row).  The caller waits for the loads (vmcnt) and synchronises before reading.
template <int D>
DKV_DEVICE void dma_rope_table(const float* __restrict__ table, const int* pos_s, float* dst) {
  constexpr int HALF_D = D / 2;
  constexpr int NC = HALF_D / 4;                       // 16-byte pieces per token
  constexpr int PER_WAVE = kTileTok * NC / 64 / (kK2Threads / 64);  // instructions per wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int S0 = (wave * PER_WAVE + i) * 64;
    const int sl = S0 + lane;
    const int n = sl / NC, c = (sl % NC) ^ (n % NC);
    __builtin_amdgcn_global_load_lds(table + (long)pos_s[n] * HALF_D + 4 * c, dst + 4 * S0, 16, 0, 0);
  }
}

// The swizzled piece of dma_rope_table holding floats 4c .. 4c + 3 of token n.
template <int D>
DKV_DEVICE int rope_piece(int n, int c) {
  constexpr int NC = D / 8;
  return n * NC + (c ^ (n % NC));
}

// DMA (decoding): the cos rows were loaded into LDS at byte offset kDmaCosOffset during the main
// loop's last groups (dma_rope_table); the sin rows go to offset 0 here, and the reads follow the
// swizzled layout.  Otherwise both are staged by stage_rope_rows.
constexpr int kDmaCosOffset = 2 * kTileTok * kStride * 2;  // bytes: past the two basis blocks

template <int D, bool ROWMAJOR, bool DMA = false>
DKV_DEVICE void keys_scores_small_epilogue(const K2Args& a, floatx16 (&acc)[2][4], half_t* lds_h,
                                           float (*stat_m)[4][32], float (*stat_s)[4][32], int tok0, int count,
                                           int tile, int h0, int b, int RH, const int* pos_s, const float* qs) {
  constexpr int HPW = 256 / D;
  constexpr int DB = D / 32;
  constexpr int HALF_BLK = DB / 2;
  constexpr int HALF_D = D / 2;
  constexpr int CSTR = HALF_D + 4;  // floats per staged RoPE row (keeps b128 reads conflict-free)
  float* cs = DMA ? (float*)((char*)lds_h + kDmaCosOffset) : (float*)lds_h;  // cos: [256][CSTR] or swizzled
  float* sn = DMA ? (float*)lds_h : cs + kTileTok * CSTR;                    // sin
  // pos_s (the tile's positions) and qs ([HPW][kSmallRows][D] query rows) were staged at kernel start
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tq = wave & 3, hs = wave >> 2;
  const int l32 = lane & 31, lhi = lane >> 5;

  if constexpr (DMA) {
    dma_rope_table<D>(a.rope_sin, pos_s, sn);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's table loads (cos and sin) have landed
    __syncthreads();
  } else {
    stage_rope_rows<D>(a, cs, sn, pos_s, count);
  }

  // part[hw][r][tb]: partial q . k over this lane's dimensions, head hw of the wave
  constexpr int HPWAVE = HPW / 2;
  float part[HPWAVE][kSmallRows][2];
#pragma unroll
  for (int hw = 0; hw < HPWAVE; ++hw)
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) part[hw][r][0] = part[hw][r][1] = 0.0f;
  // loop order: the query rows of a (row block, v4) slice are read once and serve both token blocks
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    if ((rb % DB) >= HALF_BLK) continue;
    const int rb2 = rb + HALF_BLK;
    const int hw = rb / DB;
    const int hl = hs * HPWAVE + hw;
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const int j = (rb % DB) * 32 + 8 * v4 + 4 * lhi;  // pair index, 0 .. D/2-1
      float4 qlo[kSmallRows], qhi[kSmallRows];
#pragma unroll
      for (int r = 0; r < kSmallRows; ++r) {
        if (r >= RH) break;
        qlo[r] = *(const float4*)(qs + (hl * kSmallRows + r) * D + j);
        qhi[r] = *(const float4*)(qs + (hl * kSmallRows + r) * D + j + HALF_D);
      }
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        const int n = tq * 64 + tb * 32 + l32;
        const int o = DMA ? 4 * rope_piece<D>(n, j / 4) : n * CSTR + j;
        const float4 c4 = *(const float4*)(cs + o);
        const float4 s4 = *(const float4*)(sn + o);
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
        float rlo[4], rhi[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float klo = acc[tb][rb][v4 * 4 + e];
          const float khi = acc[tb][rb2][v4 * 4 + e];
          rlo[e] = klo * cv[e] - khi * sv[e];
          rhi[e] = khi * cv[e] + klo * sv[e];
        }
#pragma unroll
        for (int r = 0; r < kSmallRows; ++r) {
          if (r >= RH) break;
          part[hw][r][tb] += qlo[r].x * rlo[0] + qlo[r].y * rlo[1] + qlo[r].z * rlo[2] + qlo[r].w * rlo[3] +
                             qhi[r].x * rhi[0] + qhi[r].y * rhi[1] + qhi[r].z * rhi[2] + qhi[r].w * rhi[3];
        }
      }
    }
  }
  // combine the two dimension halves (lanes l32 and l32 + 32), write scores, tile statistics
  float xs[HPWAVE][kSmallRows][2];
#pragma unroll
  for (int hw = 0; hw < HPWAVE; ++hw) {
    const int hl = hs * HPWAVE + hw;
    const int h = h0 + hl;
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) {
      if (r >= RH) break;
      float x[2];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        const float full = sum_xor32(part[hw][r][tb]);  // the lane's and its partner's dimension halves
        const int n = tq * 64 + tb * 32 + l32;
        x[tb] = n < count ? full * a.scaling : -INFINITY;
        xs[hw][r][tb] = x[tb];
      }
      if constexpr (ROWMAJOR) {  // question scoring: this wave's quarter (64 tokens), written at once
        const float mq = max32(fmaxf(x[0], x[1]));
        const float e0 = mq == -INFINITY ? 0.0f : __expf(x[0] - mq);
        const float e1 = mq == -INFINITY ? 0.0f : __expf(x[1] - mq);
        const float sq = sum32(e0 + e1);
        const long r_all = (long)h * RH + r;
        // lanes l32 and l32 + 32 hold both token blocks: each writes its own
        a.probs[r_all * ((long)a.ntiles * kTileTok) + (long)tile * kTileTok + tq * 64 + lhi * 32 + l32] =
            f16_bits(lhi ? e1 : e0);
        if (lane == 0) {
          a.sub_max[sub_index(r_all, tile * 4 + tq, a.ntiles * 4)] = mq;
          a.sub_sum[sub_index(r_all, tile * 4 + tq, a.ntiles * 4)] = sq;
        }
        continue;
      }
      const float mx = max32(fmaxf(x[0], x[1]));
      float sm = 0.0f;
      if (mx != -INFINITY) sm = __expf(x[0] - mx) + __expf(x[1] - mx);
      sm = sum32(sm);
      if (lane == 0) {
        stat_m[hl][tq][r] = mx;
        stat_s[hl][tq][r] = sm;
      }
    }
  }
  if constexpr (ROWMAJOR) return;  // the loop above wrote everything
  __syncthreads();
  if (tid < HPW * kSmallRows) {
    const int hl = tid / kSmallRows, r = tid % kSmallRows;
    if (r < RH) {
      float M = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; ++q) M = fmaxf(M, stat_m[hl][q][r]);
      float S = 0.0f;
      if (M != -INFINITY) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float mq = stat_m[hl][q][r];
          if (mq != -INFINITY) S += stat_s[hl][q][r] * __expf(mq - M);
        }
      }
      const long o = (long)((h0 + hl) * RH + r) * a.nstats + tile;
      a.tile_max[o] = M;
      a.tile_sum[o] = S;
    }
  }
  // probabilities relative to the tile maximum, fp16, for the value side; every slot of the
  // tile is written (0 past the tile's tokens)
  if (!a.probs) return;
#pragma unroll
  for (int hw = 0; hw < HPWAVE; ++hw) {
    const int hl = hs * HPWAVE + hw;
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r) {
      if (r >= RH) break;
      float M = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; ++q) M = fmaxf(M, stat_m[hl][q][r]);
      const float x = xs[hw][r][lhi];
      const float p = (x == -INFINITY) ? 0.0f : __expf(x - M);
      const int n = tq * 64 + lhi * 32 + l32;
      a.probs[prob_index((long)(h0 + hl) * RH + r, (long)tile * kTileTok + n, a.Hq * a.q_len)] = f16_bits(p);
    }
  }
}

// ---------------------------------------------------------------------------
// K2.  D = head_dim (64 or 128).  The workgroup covers 256 tokens x HPW =
// 256 / D heads (256 basis rows); wave w takes tokens (w & 3) * 64 .. +64
// and basis rows (w >> 2) * 128 .. +128 of the tile.  Per 64-component
// group: the decoded coefficient block [256][64] and the basis block
// [256][64] are fetched into registers one group ahead and stored into a
// double-buffered, padded LDS tile; 32x32x16 fp16 MFMAs accumulate the keys.
// ---------------------------------------------------------------------------
template <int D, bool SMALL, bool ROWMAJOR = false>
__global__ __launch_bounds__(kK2Threads) void keys_scores_kernel(K2Args a) {
  constexpr int HPW = 256 / D;      // heads per workgroup
  constexpr int DB = D / 32;        // 32-row blocks per head
  constexpr int HALF_BLK = DB / 2;  // RoPE partner offset in blocks
  __shared__ __attribute__((aligned(16))) half_t lds[2 * 2 * kTileTok * kStride];
  __shared__ float stat_m[HPW][4][32];
  __shared__ float stat_s[HPW][4][32];
  __shared__ int pos_s[kTileTok];                  // the tile's RoPE positions
  __shared__ float q_s[HPW * kSmallRows * D];      // the workgroup's query rows (decode epilogue)

  const int bid = blockIdx.x;
  const int lin = (bid & 7) * a.per_xcd + (bid >> 3);
  if (lin >= a.total_wg) return;
  const int nhg = a.Hkv / HPW;
  const int tile = lin / nhg, hg = lin % nhg;  // consecutive ids (one XCD): the head groups of a tile
  const int2 bt = find_tile(a.cu_seqlens, a.batch, a.n_total, kTileTok, tile);
  const int b = bt.x;
  const int2 sr = seq_range(a.cu_seqlens, a.batch, a.n_total, b);
  const int tok0 = sr.x + bt.y * kTileTok;
  const int count = min(kTileTok, sr.y - tok0);
  const int h0 = hg * HPW;
  const int G = a.G;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tq = wave & 3, hs = wave >> 2;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int RH = (a.Hq / a.Hkv) * a.q_len;

  // First round, ahead of the main loop's loads: the epilogue's positions (clamped into the RoPE
  // tables; past the tile's end, its last token's) and the decode epilogue's query rows, as raw bits
  // from unconditional loads (rows past RH read row RH - 1 and are written as 0).  They reach LDS once
  // the main loop's first loads are out: storing each as it arrives, or converting under a type
  // switch, made every later load wait for it.
  const int pos_raw = a.positions[tok0 + min(tid % kTileTok, count - 1)];
  constexpr int QE = SMALL ? HPW * kSmallRows * D / kK2Threads : 1;  // query elements per thread
  static_assert(!SMALL || QE * kK2Threads == HPW * kSmallRows * D, "whole rounds of query elements");
  const bool q32 = a.query_dtype == DKV_F32;
  uint32_t qlo_bits[QE], qhi_bits[QE];
  if constexpr (SMALL) {
    const int gq = a.Hq / a.Hkv;
#pragma unroll
    for (int i = 0; i < QE; ++i) {
      const int e = tid + i * kK2Threads;
      const int hl = e / (kSmallRows * D), r = min((e / D) % kSmallRows, RH - 1), d = e % D;
      const int qh = (h0 + hl) * gq + r / a.q_len, qi = r % a.q_len;
      const long idx = (((long)b * a.Hq + qh) * a.q_len + qi) * D + d;
      const uint16_t* qp = (const uint16_t*)a.query + (q32 ? 2 * idx : idx);
      qlo_bits[i] = qp[0];
      qhi_bits[i] = qp[q32 ? 1 : 0];
    }
  }
  auto write_first_round = [&]() {
    if (tid < kTileTok) pos_s[tid] = min(max(pos_raw, 0), a.rope_rows - 1);
    if constexpr (SMALL) {
#pragma unroll
      for (int i = 0; i < QE; ++i) {
        const int e = tid + i * kK2Threads;
        const float qv = q32 ? __uint_as_float(qlo_bits[i] | qhi_bits[i] << 16)
                             : a.query_dtype == DKV_F16 ? half_bits_to_float((uint16_t)qlo_bits[i])
                                                        : bf16_bits_to_float((uint16_t)qlo_bits[i]);
        q_s[e] = (e / D) % kSmallRows < RH ? qv : 0.0f;
      }
    }
  };

  // Coefficient operands come straight from the decoded buffer (one 16-byte
  // load per lane per MFMA operand); the basis block [256][64] goes global ->
  // registers -> padded, double-buffered LDS, each row half by its own waves.
  // Both are fetched ahead (coefficients three segments, basis two).
  const half8* coef_frag = (const half8*)a.coef + ((long)(tile * 8 + tq * 2) * 4) * 64 + lane;
  const long coef_group_stride = (long)(a.n_slots / 32) * 4 * 64;  // in half8 units
  const uint16_t* basis_layer = a.key_basis + (long)a.layer * G * a.Hkv * D * 64 + (long)h0 * D * 64;
  const long basis_group_stride = (long)a.Hkv * D * 64;

  half_t* B0 = lds;  // basis [2][256][72]
  const int gt = tid & 255;  // thread within its row half

  const float* mean_rows = a.mean_k + ((long)a.layer * a.Hkv + h0) * D + hs * 128 + 4 * lhi;
  floatx16 acc[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const float4 m4 = *(const float4*)(mean_rows + j * 32 + 8 * v4);
      acc[0][j][4 * v4 + 0] = acc[1][j][4 * v4 + 0] = m4.x;
      acc[0][j][4 * v4 + 1] = acc[1][j][4 * v4 + 1] = m4.y;
      acc[0][j][4 * v4 + 2] = acc[1][j][4 * v4 + 2] = m4.z;
      acc[0][j][4 * v4 + 3] = acc[1][j][4 * v4 + 3] = m4.w;
    }

  // af[tb*4 + ks]: coefficient operand of token block tb, step ks
  half8 af0[8], af1[8];
  uint4 br0, br1, br2, br3;

#define DKV_K2_ISSUE_A(g_, af_)                                             \
  do {                                                                      \
    const half8* src_ = coef_frag + (long)(g_) * coef_group_stride;        \
    af_[0] = src_[0 * 64]; af_[1] = src_[1 * 64]; af_[2] = src_[2 * 64];   \
    af_[3] = src_[3 * 64]; af_[4] = src_[4 * 64]; af_[5] = src_[5 * 64];   \
    af_[6] = src_[6 * 64]; af_[7] = src_[7 * 64];                          \
  } while (0)

#define DKV_K2_ISSUE_B(g_)                                                            \
  do {                                                                                \
    const uint4* src_ = (const uint4*)(basis_layer + (long)(g_) * basis_group_stride) + hs * 1024; \
    br0 = src_[0 * 256 + gt];                                                         \
    br1 = src_[1 * 256 + gt];                                                         \
    br2 = src_[2 * 256 + gt];                                                         \
    br3 = src_[3 * 256 + gt];                                                         \
  } while (0)

#define DKV_K2_STORE(dst_, j_, v_) \
  *(uint4*)((dst_) + (hs * 128 + (((j_) * 256 + gt) >> 3)) * kStride + (gt & 7) * 8) = (v_)

#define DKV_K2_FINISH(buf_)                                \
  do {                                                     \
    half_t* bdst_ = B0 + (buf_) * kTileTok * kStride;      \
    DKV_K2_STORE(bdst_, 0, br0);                           \
    DKV_K2_STORE(bdst_, 1, br1);                           \
    DKV_K2_STORE(bdst_, 2, br2);                           \
    DKV_K2_STORE(bdst_, 3, br3);                           \
  } while (0)

#define DKV_K2_MFMA(buf_, af_)                                                         \
  do {                                                                                 \
    const half_t* Bt = B0 + (buf_) * kTileTok * kStride;                               \
    _Pragma("unroll") for (int ks = 0; ks < 4; ++ks) {                                 \
      const int kof = ks * 16 + lhi * 8;                                               \
      half8 aop[4];                                                                    \
      _Pragma("unroll") for (int rb = 0; rb < 4; ++rb)                                 \
        aop[rb] = lds_half8(Bt + (hs * 128 + rb * 32 + l32) * kStride + kof);          \
      _Pragma("unroll") for (int tb = 0; tb < 2; ++tb)                                 \
        _Pragma("unroll") for (int rb = 0; rb < 4; ++rb)                               \
          acc[tb][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[rb], af_[tb * 4 + ks], acc[tb][rb], 0, 0, 0); \
    }                                                                                  \
  } while (0)

  // Main loop, two groups per iteration.  Ping-pong: the two row
  // halves (waves 0-3 and 4-7, one of each on every SIMD) each load and read
  // only their own 128 basis rows, and alternate MFMA segments with memory
  // segments (LDS writes of the next block, next loads), one barrier apart:
  // half 1 starts one barrier late and half 0 ends one barrier late, so every
  // wave executes the same number of barriers and, between two barriers, one
  // wave of a SIMD runs MFMAs while the other does its memory work.
  // sched_barrier keeps the compiler from moving loads into the MFMA
  // segments; a wave in its MFMA segment runs at raised priority.
  // prologue: group 0's basis first (the LDS store waits for it alone), its coefficient operands in
  // k-step order (the first MFMAs wait for the first two), group 1's operands, then group 1's basis
  // (its registers are free once group 0's block is stored)
  DKV_K2_ISSUE_B(0);
  {
    const half8* src_ = coef_frag;
    af0[0] = src_[0 * 64]; af0[4] = src_[4 * 64]; af0[1] = src_[1 * 64]; af0[5] = src_[5 * 64];
    af0[2] = src_[2 * 64]; af0[6] = src_[6 * 64]; af0[3] = src_[3 * 64]; af0[7] = src_[7 * 64];
  }
  DKV_K2_ISSUE_A(1, af1);
  __builtin_amdgcn_sched_barrier(0);
  write_first_round();
  DKV_K2_FINISH(0);
  DKV_K2_ISSUE_B(1);
  __syncthreads();
  if (hs == 1) __builtin_amdgcn_s_barrier();
  // G is even (the rank is a multiple of 256).  The last two groups run
  // after the loop, which loads nothing more: loads past the end would only repeat the last group and
  // hold up the epilogue's loads behind them (a branch around them in the loop costs more: the
  // compiler then waits for every load at the join).
  for (int g = 0; g < G - 2; g += 2) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    DKV_K2_MFMA(0, af0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    DKV_K2_FINISH(1);
    DKV_K2_ISSUE_B(g + 2);
    DKV_K2_ISSUE_A(g + 2, af0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    DKV_K2_MFMA(1, af1);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    DKV_K2_FINISH(0);
    DKV_K2_ISSUE_B(g + 3);
    DKV_K2_ISSUE_A(g + 3, af1);
    __syncthreads();
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(1);
  DKV_K2_MFMA(0, af0);
  __builtin_amdgcn_s_setprio(0);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  DKV_K2_FINISH(1);
  // the tile's cos rows go straight to LDS past the basis blocks while the last MFMAs run (every
  // epilogue but the few-row scoring one, which stages its rows itself)
  if constexpr (!(SMALL && ROWMAJOR)) dma_rope_table<D>(a.rope_cos, pos_s, (float*)((char*)lds + kDmaCosOffset));
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(1);
  DKV_K2_MFMA(1, af1);
  __builtin_amdgcn_s_setprio(0);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __syncthreads();
  if (hs == 0) __builtin_amdgcn_s_barrier();
#undef DKV_K2_ISSUE_A
#undef DKV_K2_ISSUE_B
#undef DKV_K2_MFMA
#undef DKV_K2_STORE
#undef DKV_K2_FINISH
  __syncthreads();

  const int gq = a.Hq / a.Hkv;
  if constexpr (SMALL) {
    keys_scores_small_epilogue<D, ROWMAJOR, !ROWMAJOR>(a, acc, lds, stat_m, stat_s, tok0, count, tile, h0, b, RH,
                                                       pos_s, q_s);
    return;
  } else {

  // ---- epilogue 1 (many query rows): RoPE in registers, straight into MFMA key fragments.  The
  // tile's cos / sin rows are in LDS (dma_rope_table: cos during the last groups, sin here); each lane rotates the
  // (d, d + D/2) pairs it holds in fp32 and rounds them to fp16.  Lane (l32, lhi) then holds, for
  // its token, 4 of the 8 dimensions of every 8-dimension chunk c (offset 4 lhi); the key fragment
  // of k-step ks needs chunk 2 ks + lhi whole, which one permlane32 swap per dword of the chunk pair
  // (2 ks, 2 ks + 1) provides: lanes 0-31 keep their chunk 2 ks half and get lanes 32-63's, lanes
  // 32-63 keep their chunk 2 ks + 1 half and get lanes 0-31's.
  constexpr int HPWAVE = HPW / 2;  // heads handled by each wave in the epilogue
  constexpr int KS = D / 16;       // MFMA k-steps over the head dimension
  half8 kf[HPWAVE][KS][2];
  {
    const float* cs = (const float*)((const char*)lds + kDmaCosOffset);
    float* sn = (float*)lds;
    dma_rope_table<D>(a.rope_sin, pos_s, sn);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's table loads (cos and sin) have landed
    __syncthreads();
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const int n = tq * 64 + tb * 32 + l32;
      uint32_t own[HPWAVE][D / 8][2];  // chunk c of head hh: this lane's 4 halves as 2 dwords
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        if ((rb % DB) >= HALF_BLK) continue;
        const int rb2 = rb + HALF_BLK;
        const int hh = rb / DB;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const int d0 = (rb % DB) * 32 + 8 * v4 + 4 * lhi;
          const int o = 4 * rope_piece<D>(n, d0 / 4);
          const float4 c4 = *(const float4*)(cs + o);
          const float4 s4 = *(const float4*)(sn + o);
          const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
          const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
          uint32_t lo[2], hi[2];
#pragma unroll
          for (int e = 0; e < 4; e += 2) {
            const float klo0 = acc[tb][rb][v4 * 4 + e], khi0 = acc[tb][rb2][v4 * 4 + e];
            const float klo1 = acc[tb][rb][v4 * 4 + e + 1], khi1 = acc[tb][rb2][v4 * 4 + e + 1];
            lo[e / 2] = pack_f16x2(klo0 * cv[e] - khi0 * sv[e], klo1 * cv[e + 1] - khi1 * sv[e + 1]);
            hi[e / 2] = pack_f16x2(khi0 * cv[e] + klo0 * sv[e], khi1 * cv[e + 1] + klo1 * sv[e + 1]);
          }
          const int clo = (rb % DB) * 4 + v4, chi = (rb2 % DB) * 4 + v4;
          own[hh][clo][0] = lo[0];
          own[hh][clo][1] = lo[1];
          own[hh][chi][0] = hi[0];
          own[hh][chi][1] = hi[1];
        }
      }
#pragma unroll
      for (int hh = 0; hh < HPWAVE; ++hh)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const auto w0 = __builtin_amdgcn_permlane32_swap(own[hh][2 * ks][0], own[hh][2 * ks + 1][0], false, false);
          const auto w1 = __builtin_amdgcn_permlane32_swap(own[hh][2 * ks][1], own[hh][2 * ks + 1][1], false, false);
          const uint32_t f[4] = {w0[0], w1[0], w0[1], w1[1]};
          __builtin_memcpy(&kf[hh][ks][tb], f, 16);
        }
    }
  }
  // the staged RoPE rows are read by every wave before any reuses their LDS
  __syncthreads();

  // ---- epilogue 2: scores = q . k * scaling on MFMA, per 32-row block, with the key fragments in
  // registers; the query fragments of a row block are loaded together (rows past the end read the
  // last row, whose scores are discarded), in the query's own type.
  const int mblocks = (RH + 31) / 32;
  // the query fragments of row block mb of head h (rows past the end read the last row)
  auto load_queries = [&](auto qtype, auto (&qf)[KS], int h, int mb) {
    constexpr int QT = decltype(qtype)::value;
    const int r = min(mb * 32 + l32, RH - 1);
    const int qh = h * gq + r / a.q_len, qi = r % a.q_len;
    const long qbase = (((long)b * a.Hq + qh) * a.q_len + qi) * D + lhi * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = load_query_frag<QT>(a.query, qbase + ks * 16);
  };
  // sacc[tb][v] = q . k for token tq*64 + tb*32 + l32 and row mb*32 + 8*(v/4) + 4*lhi + (v&3), or,
  // with the operands exchanged (TOKENS_IN_V), for token tq*64 + tb*32 + 8*(v/4) + 4*lhi + (v&3) and
  // row mb*32 + l32
  auto block_mfma = [&](auto qtype, auto tokens_in_v, floatx16 (&sacc)[2], const half8 (&kf)[KS][2],
                        const auto (&qf)[KS]) {
    constexpr int QT = decltype(qtype)::value;
    constexpr bool TOKENS_IN_V = decltype(tokens_in_v)::value;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int v = 0; v < 16; ++v) sacc[tb][v] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const half8 q8 = query_frag_half<QT>(qf[ks]);
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        if constexpr (TOKENS_IN_V)
          sacc[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks][tb], q8, sacc[tb], 0, 0, 0);
        else
          sacc[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(q8, kf[ks][tb], sacc[tb], 0, 0, 0);
      }
    }
  };

  // question scoring: probabilities relative to this wave's 64 tokens (a tile quarter) and the
  // quarter's (max, sum), written at once: no exchange between waves, so heads and row blocks run in
  // any order (heads outer: one head's key fragments in registers at a time).  The scores come with
  // the tokens in the accumulator registers and the rows across the lanes, so a row's quarter
  // statistics are 32 values in the lane and one exchange with lane l32 + 32.
  // The workgroup's query rows go to LDS once, as fp16, in chunks of up to QROWS rows per head: the
  // four token quarters of a head read the same rows, which loaded per wave would cross each CU's
  // load path four times.
  auto row_blocks_quarters = [&](auto qtype) {
    constexpr int QT = decltype(qtype)::value;
    // each wave stages its probabilities in LDS so that every global store writes whole 128-byte lines
    constexpr int SROW = 72;                                // staging row: 64 tokens + 8 halves of padding
    constexpr int QSTR = D + 8;                             // staged query row (conflict-free b128 reads)
    constexpr int LDS_HALVES = 2 * 2 * kTileTok * kStride;  // the lds array
    constexpr int STAGE_HALVES = (kK2Threads / 64) * 32 * SROW;
    constexpr int QROWS = (LDS_HALVES - STAGE_HALVES) / (HPW * QSTR) / 32 * 32;  // 192 at D = 64 and 128
    static_assert(QROWS >= 32, "query chunk");
    constexpr int C8 = D / 8;             // 8-element pieces per query row
    constexpr int RPP = kK2Threads / C8;  // rows per staging pass
    constexpr int PPH = QROWS / RPP;      // passes per head
    static_assert(QROWS % RPP == 0, "staging passes");
    half_t* qlds = lds;  // [HPW][QROWS][QSTR]
    half_t* stage = lds + HPW * QROWS * QSTR + wave * 32 * SROW;
    // this lane's piece of a staged probability row: tokens (lane & 7) * 8 .. + 8 of the wave's quarter
    const long pstride = (long)a.ntiles * kTileTok;
    uint16_t* pbase = a.probs + (long)tile * kTileTok + tq * 64 + (lane & 7) * 8;
    const long lane_row = (long)(lane >> 3) * pstride;
    const int c8 = tid % C8, rsub = tid / C8;
    // row r of head h0 + hl is query row b * Hq * q_len + (h0 + hl) * RH + r
    const long qrow0 = (long)b * a.Hq * a.q_len + (long)h0 * RH;
    for (int c0 = 0; c0 < RH; c0 += QROWS) {
      const int nblk = (min(QROWS, RH - c0) + 31) / 32;
      if (c0 > 0) __syncthreads();  // the previous chunk's rows are read (the first: the RoPE rows)
      // QROWS rows per head, rows past the end repeating row RH - 1 (their loads all hit one row's
      // lines; the rows are never read): every load unconditional and issued before any is used
      RawQuery8<QT> qv[HPW * PPH];
#pragma unroll
      for (int p = 0; p < HPW * PPH; ++p) {
        const int hl = p / PPH, rl = (p % PPH) * RPP + rsub;
        qv[p] = load_raw_query8<QT>(a.query, (qrow0 + hl * RH + min(c0 + rl, RH - 1)) * D + c8 * 8);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int p = 0; p < HPW * PPH; ++p) {
        const int hl = p / PPH, rl = (p % PPH) * RPP + rsub;
        *(half8*)(qlds + (hl * QROWS + rl) * QSTR + c8 * 8) = raw_query8_half<QT>(qv[p]);
      }
      __syncthreads();
#pragma unroll
      for (int hh = 0; hh < HPWAVE; ++hh) {
        const int hl = hs * HPWAVE + hh;
        const int h = h0 + hl;
        // the fp16 query fragments of row block mb of the chunk
        auto read_queries = [&](half8 (&qf)[KS], int mb) {
          const half_t* src = qlds + (hl * QROWS + mb * 32 + l32) * QSTR + lhi * 8;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) qf[ks] = lds_half8(src + ks * 16);
        };
        auto quarter = [&](const half8 (&qf)[KS], int mb) {
          floatx16 sacc[2];
          block_mfma(QueryType<DKV_F32>{}, QueryType<1>{}, sacc, kf[hh], qf);  // fp16 fragments as they are
          // The maximum is taken over the raw dot products (the scale is positive) and the scale folds
          // into the exponent: p = 2^(q.k * scale * log2(e) - max * scale * log2(e)), one fma and one
          // exp2 per score.  Tokens past the tile's end (last tile only) score -inf.
          if (count < kTileTok) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int n = tq * 64 + tb * 32 + 8 * (v >> 2) + 4 * lhi + (v & 3);
                sacc[tb][v] = n < count ? sacc[tb][v] : -INFINITY;
              }
          }
          float mraw = -INFINITY;
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int v = 0; v < 16; ++v) mraw = fmaxf(mraw, sacc[tb][v]);
          mraw = max_xor32(mraw);
          const float c2 = a.scaling * 1.44269504088896341f;
          const float off2 = mraw == -INFINITY ? 0.0f : mraw * c2;
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              sacc[tb][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[tb][v], c2, -off2));  // -inf -> 0
          const float mx = mraw * a.scaling;  // the quarter maximum of the scaled scores (-inf if empty)
          const int row0 = c0 + mb * 32;      // first row of the block
          // the fp16 probabilities: pw[tb][j] holds tokens tb*32 + 8j + 4lhi .. + 3 of row l32
          uint2 pw[2][4];
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              pw[tb][j] = make_uint2(pack_f16x2(sacc[tb][4 * j], sacc[tb][4 * j + 1]),
                                     pack_f16x2(sacc[tb][4 * j + 2], sacc[tb][4 * j + 3]));
          // the quarter sum of the fp32 probabilities (lanes l32 and l32 + 32 hold the row's halves)
          float sm = 0.0f;
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int v = 0; v < 16; ++v) sm += sacc[tb][v];
          sm = sum_xor32(sm);
          // row l32 of the block into the staging rows
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 4; ++j) *(uint2*)(stage + l32 * SROW + tb * 32 + 8 * j + 4 * lhi) = pw[tb][j];
          __builtin_amdgcn_wave_barrier();  // LDS runs a wave's accesses in order: the reads see the writes
          // lane L then holds 8 tokens of rows L/8 + 8k: eight lanes write one row's 128 bytes.  In the
          // last, partial block rows past the end were computed from row RH - 1's query and key bits,
          // so they store the same bytes there.
          typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
          u32x4 pv[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) pv[k] = *(const u32x4*)(stage + ((lane >> 3) + 8 * k) * SROW + (lane & 7) * 8);
          // the four reads go out together, ahead of the branch (the compiler would otherwise read and
          // wait once per store inside it)
          asm volatile("" ::"v"(pv[0]), "v"(pv[1]), "v"(pv[2]), "v"(pv[3]));
          if (row0 + 32 <= RH) {  // a whole block: rows row0 + (lane >> 3) + 8 k, 8 rows apart
            uint16_t* dst = pbase + (long)(h * RH + row0) * pstride + lane_row;
#pragma unroll
            for (int k = 0; k < 4; ++k) *(u32x4*)(dst + 8 * k * pstride) = pv[k];
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const long r = (long)h * RH + min(row0 + (lane >> 3) + 8 * k, RH - 1);
              *(u32x4*)(pbase + r * pstride) = pv[k];
            }
          }
          __builtin_amdgcn_wave_barrier();  // the next block's staging writes stay behind these reads
          // lanes l32 and l32 + 32 hold the same statistics
          const long r_all = (long)h * RH + min(row0 + l32, RH - 1);
          a.sub_max[sub_index(r_all, tile * 4 + tq, a.ntiles * 4)] = mx;
          a.sub_sum[sub_index(r_all, tile * 4 + tq, a.ntiles * 4)] = sm;
        };
        // two fragment buffers: the next row block's fragments are read while this block's MFMAs run
        half8 qa[KS], qb[KS];
        read_queries(qa, 0);
        for (int mb = 0; mb < nblk; mb += 2) {
          read_queries(qb, min(mb + 1, nblk - 1));
          __builtin_amdgcn_sched_barrier(0);
          quarter(qa, mb);
          if (mb + 1 >= nblk) break;
          read_queries(qa, min(mb + 2, nblk - 1));
          __builtin_amdgcn_sched_barrier(0);
          quarter(qb, mb + 1);
        }
      }
    }
  };

  // decoding many rows: the four waves of a head exchange their quarters' statistics per row block,
  // then write probabilities relative to the tile maximum in the value side's layout
  auto row_blocks = [&](auto qtype) {
    for (int mb = 0; mb < mblocks; ++mb) {
      float xs[HPWAVE][16][2];
#pragma unroll
      for (int hh = 0; hh < HPWAVE; ++hh) {
        const int hl = hs * HPWAVE + hh;
        typename QueryFrag<decltype(qtype)::value>::type qf[KS];
        load_queries(qtype, qf, h0 + hl, mb);
        __builtin_amdgcn_sched_barrier(0);
        floatx16 sacc[2];
        block_mfma(qtype, QueryType<0>{}, sacc, kf[hh], qf);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = mb * 32 + 8 * (v >> 2) + 4 * lhi + (v & 3);
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) {
            const int n = tq * 64 + tb * 32 + l32;
            xs[hh][v][tb] = (row < RH) && (n < count) ? sacc[tb][v] * a.scaling : -INFINITY;
          }
          const float mx = max32(fmaxf(xs[hh][v][0], xs[hh][v][1]));
          float sm = 0.0f;
          if (mx != -INFINITY) sm = __expf(xs[hh][v][0] - mx) + __expf(xs[hh][v][1] - mx);
          sm = sum32(sm);
          if (l32 == 0) {
            const int rr = 8 * (v >> 2) + 4 * lhi + (v & 3);
            stat_m[hl][tq][rr] = mx;
            stat_s[hl][tq][rr] = sm;
          }
        }
      }
      __syncthreads();
      if (tid < HPW * 32) {
        const int hl = tid >> 5, rr = tid & 31;
        const int row = mb * 32 + rr;
        if (row < RH) {
          float M = -INFINITY;
#pragma unroll
          for (int q = 0; q < 4; ++q) M = fmaxf(M, stat_m[hl][q][rr]);
          float S = 0.0f;
          if (M != -INFINITY) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float mq = stat_m[hl][q][rr];
              if (mq != -INFINITY) S += stat_s[hl][q][rr] * __expf(mq - M);
            }
          }
          const long o = (long)((h0 + hl) * RH + row) * a.nstats + tile;
          a.tile_max[o] = M;
          a.tile_sum[o] = S;
        }
      }
      // probabilities relative to the tile maximum (fp16), from the registers; 0 past the tokens
#pragma unroll
      for (int hh = 0; hh < HPWAVE; ++hh) {
        const int hl = hs * HPWAVE + hh;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rr = 8 * (v >> 2) + 4 * lhi + (v & 3);
          const int row = mb * 32 + rr;
          if (row >= RH) continue;
          float M = -INFINITY;
#pragma unroll
          for (int q = 0; q < 4; ++q) M = fmaxf(M, stat_m[hl][q][rr]);
          const long r_all = (long)(h0 + hl) * RH + row;
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) {
            const float x = xs[hh][v][tb];
            const int n = tq * 64 + tb * 32 + l32;
            a.probs[prob_index(r_all, (long)tile * kTileTok + n, a.Hq * a.q_len)] =
                f16_bits(x == -INFINITY ? 0.0f : __expf(x - M));
          }
        }
      }
      __syncthreads();
    }
  };
  if constexpr (ROWMAJOR) {
    if (a.query_dtype == DKV_F16)
      row_blocks_quarters(QueryType<DKV_F16>{});
    else if (a.query_dtype == DKV_BF16)
      row_blocks_quarters(QueryType<DKV_BF16>{});
    else
      row_blocks_quarters(QueryType<DKV_F32>{});
  } else {
    if (a.query_dtype == DKV_F16)
      row_blocks(QueryType<DKV_F16>{});
    else if (a.query_dtype == DKV_BF16)
      row_blocks(QueryType<DKV_BF16>{});
    else
      row_blocks(QueryType<DKV_F32>{});
  }
  }
}

// ---------------------------------------------------------------------------
// K2, one KV head per workgroup: decoding contexts whose 256-row workgroups
// (256 / D heads each) would leave CUs idle, but whose (tile, head) pairs fill
// them.  The workgroup covers the tile's 256 tokens and the head's D basis
// rows over every 64-component group, so no partial scores are merged
// afterwards and the tile statistics, probabilities and their layouts are the
// 256-row kernel's.  Wave w takes the tile's 32-token block w: its coefficient
// operands come straight from the decoded buffer (four 16-byte loads per lane
// and group) and the head's basis blocks [D][64] go global -> registers ->
// LDS (D / 64 16-byte loads per thread and group), with the loads of four
// groups in flight.  One group per barrier: group g's basis block goes to LDS
// block g & 1, whose previous readers (group g - 2) finished before the
// barrier of group g - 1.  Consecutive workgroup ids (one XCD) are the heads
// of one tile, which read the same coefficients.
// ---------------------------------------------------------------------------

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>), in order
template <class Fn, int... Is>
DKV_DEVICE void static_for_seq(Fn&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class Fn>
DKV_DEVICE void static_for(Fn&& f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// NW waves of 32 tokens: the whole tile (8), or half of it (4) when short contexts leave CUs idle
// even with one workgroup per (tile, head); the softmax statistics then cover the workgroup's 128
// tokens (entry 2 * tile + half).
template <int D, int NW>
__global__ __launch_bounds__(NW * 64) void keys_scores_head_kernel(K2Args a) {
  constexpr int NT = NW * 64;       // threads
  constexpr int TT = NW * 32;       // tokens of the workgroup
  constexpr int PARTS = kTileTok / TT;
  constexpr int DB = D / 32;        // 32-row blocks of the head
  constexpr int HALF_BLK = DB / 2;  // RoPE partner offset in blocks
  constexpr int HALF_D = D / 2;
  constexpr int BQ = D * 8 / NT;    // basis loads per thread and group: [D][64] fp16 = D * 8 x 16 B
  constexpr int RING = 4;           // groups whose loads are in flight
  constexpr int BLK = D * kStride;  // halves per LDS basis block
  constexpr int QE = (kSmallRows * D + NT - 1) / NT;  // query elements per thread
  static_assert(NW == 8 || NW == 4, "a tile or half of it");
  static_assert(BQ * NT == D * 8, "whole rounds of basis loads");
  __shared__ __attribute__((aligned(16))) half_t lds[2 * BLK];  // two basis blocks
  __shared__ __attribute__((aligned(16))) float stat_m[NW][kSmallRows];
  __shared__ __attribute__((aligned(16))) float stat_s[NW][kSmallRows];
  __shared__ __attribute__((aligned(16))) float q_s[kSmallRows * D];  // rows past RH are 0

  const int lin = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (lin >= a.total_wg) return;
  const int tp = lin / a.Hkv, h = lin % a.Hkv;  // tp = PARTS * tile + part: the statistics entry
  const int tile = tp / PARTS, part = tp % PARTS;
  const int2 bt = find_tile(a.cu_seqlens, a.batch, a.n_total, kTileTok, tile);
  const int b = bt.x;
  const int2 sr = seq_range(a.cu_seqlens, a.batch, a.n_total, b);
  const int tok0 = sr.x + bt.y * kTileTok;
  const int count = min(kTileTok, sr.y - tok0);
  const int G = a.G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int gq = a.Hq / a.Hkv;
  const int RH = gq * a.q_len;
  const int n = part * TT + wave * 32 + l32;  // the lane's token in the tile

  // First round, before the main loop's loads: the lane's position (clamped into the RoPE tables;
  // past the tile's end, its last token's), one query element per thread and the key mean rows.
  // Their LDS copies are written once the main loop's first loads are out.
  const int pos = min(max(a.positions[tok0 + min(n, count - 1)], 0), a.rope_rows - 1);
  // the query elements as raw bits from two unconditional 16-bit loads each (a float's halves, or the
  // same 16-bit element twice), converted after the main loop's loads are out: loads under a type
  // switch made the conversion wait for the value before anything else was issued
  const bool q32 = a.query_dtype == DKV_F32;
  uint32_t qlo_bits[QE], qhi_bits[QE];
#pragma unroll
  for (int i = 0; i < QE; ++i) {
    const int e = min(tid + i * NT, kSmallRows * D - 1);
    const int qrc = min(e / D, RH - 1), qd = e % D;
    const long qi = (((long)b * a.Hq + h * gq + qrc / a.q_len) * a.q_len + qrc % a.q_len) * D + qd;
    const uint16_t* qp = (const uint16_t*)a.query + (q32 ? 2 * qi : qi);
    qlo_bits[i] = qp[0];
    qhi_bits[i] = qp[q32 ? 1 : 0];
  }
  // acc[rb][v]: basis row rb * 32 + 8 (v / 4) + 4 lhi + (v & 3) of the lane's token, from the key mean
  const float* mean_rows = a.mean_k + ((long)a.layer * a.Hkv + h) * D + 4 * lhi;
  floatx16 acc[DB];
#pragma unroll
  for (int rb = 0; rb < DB; ++rb)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const float4 m4 = *(const float4*)(mean_rows + rb * 32 + 8 * v4);
      acc[rb][4 * v4 + 0] = m4.x;
      acc[rb][4 * v4 + 1] = m4.y;
      acc[rb][4 * v4 + 2] = m4.z;
      acc[rb][4 * v4 + 3] = m4.w;
    }

  const half8* coef_frag = (const half8*)a.coef + ((long)(tile * 8 + part * NW + wave) * 4) * 64 + lane;
  const long coef_group_stride = (long)(a.n_slots / 32) * 4 * 64;  // in half8 units
  const uint4* basis_head =
      (const uint4*)(a.key_basis + (long)a.layer * G * a.Hkv * D * 64 + (long)h * D * 64) + tid;
  const long basis_group_stride = (long)a.Hkv * D * 64 / 8;  // in uint4 units

  half8 af[RING][4];  // coefficient operands of the groups in flight, per 16-component step
  // basis pieces of the groups in flight: one vector per slot (as arrays, the compiler kept them
  // in scratch memory)
  typedef uint32_t BasisVec __attribute__((ext_vector_type(4 * BQ)));
  static_assert(RING == 4, "four basis slots");
  BasisVec bq0, bq1, bq2, bq3;
  auto bq_slot = [&](auto slot) -> BasisVec& {
    constexpr int s = decltype(slot)::value;
    if constexpr (s == 0) return bq0;
    else if constexpr (s == 1) return bq1;
    else if constexpr (s == 2) return bq2;
    else return bq3;
  };
  auto issue_basis = [&](int g, auto slot) {
    BasisVec v;
#pragma unroll
    for (int i = 0; i < BQ; ++i) {
      const uint4 t = basis_head[(long)g * basis_group_stride + i * NT];
      v[4 * i] = t.x;
      v[4 * i + 1] = t.y;
      v[4 * i + 2] = t.z;
      v[4 * i + 3] = t.w;
    }
    bq_slot(slot) = v;
  };
  auto issue_coef = [&](int g, auto slot) {
    constexpr int s = decltype(slot)::value;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) af[s][ks] = coef_frag[(long)g * coef_group_stride + ks * 64];
  };
  auto store_basis = [&](auto slot) {  // slot s -> LDS block s & 1
    constexpr int s = decltype(slot)::value;
    half_t* Bt = lds + (s & 1) * BLK;
    const BasisVec v = bq_slot(slot);
#pragma unroll
    for (int i = 0; i < BQ; ++i) {
      const int e = tid + i * NT;
      *(uint4*)(Bt + (e >> 3) * kStride + (e & 7) * 8) = make_uint4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    }
  };
  // the lane's RoPE rows (pair j of dimension pairs rb * 32 + 8 v4 + 4 lhi + e, rb < HALF_BLK), as
  // 16-byte loads issued with the last groups
  float4 cw[HALF_BLK][4], sw[HALF_BLK][4];
  auto issue_rope = [&]() {
    const float* crow = a.rope_cos + (long)pos * HALF_D + 4 * lhi;
    const float* srow = a.rope_sin + (long)pos * HALF_D + 4 * lhi;
#pragma unroll
    for (int rb = 0; rb < HALF_BLK; ++rb)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        cw[rb][v4] = *(const float4*)(crow + rb * 32 + 8 * v4);
        sw[rb][v4] = *(const float4*)(srow + rb * 32 + 8 * v4);
      }
  };
  auto write_query = [&]() {
#pragma unroll
    for (int i = 0; i < QE; ++i) {
      const int e = tid + i * NT;
      const float qv = q32 ? __uint_as_float(qlo_bits[i] | qhi_bits[i] << 16)
                           : a.query_dtype == DKV_F16 ? half_bits_to_float((uint16_t)qlo_bits[i])
                                                      : bf16_bits_to_float((uint16_t)qlo_bits[i]);
      if (e < kSmallRows * D) q_s[e] = e / D < RH ? qv : 0.0f;
    }
  };
  using T = std::true_type;
  using F = std::false_type;
  // one group per barrier: its basis block into LDS block g & 1 (that block's previous readers, two
  // groups back, finished before the last barrier), a barrier, the slot's next basis loads, the
  // MFMAs (operands read from LDS), then the slot's next coefficient loads (the MFMAs have read them)
  auto group = [&](int g, auto slot, auto load_next) {
    constexpr int sl = decltype(slot)::value;
    store_basis(slot);
    __syncthreads();
    if constexpr (decltype(load_next)::value) issue_basis(g + RING, slot);
    const half_t* Bt = lds + (sl & 1) * BLK;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      half8 ao[DB];
#pragma unroll
      for (int rb = 0; rb < DB; ++rb) ao[rb] = lds_half8(Bt + (rb * 32 + l32) * kStride + ks * 16 + lhi * 8);
#pragma unroll
      for (int rb = 0; rb < DB; ++rb)
        acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ao[rb], af[sl][ks], acc[rb], 0, 0, 0);
    }
    if constexpr (decltype(load_next)::value) issue_coef(g + RING, slot);
  };
  // the first RING groups' loads in group order (left to itself, the scheduler issued group 0's
  // basis last, and the loop's first wait then covered every load in flight)
  static_for<RING>([&](auto s) {
    issue_basis(decltype(s)::value, s);
    issue_coef(decltype(s)::value, s);
    __builtin_amdgcn_sched_barrier(0);
  });
  write_query();
  // G is a multiple of RING (k2_head_form); the last RING groups load nothing more
  for (int g0 = 0; g0 < G - RING; g0 += RING) static_for<RING>([&](auto s) { group(g0 + decltype(s)::value, s, T{}); });
  issue_rope();
  static_for<RING>([&](auto s) { group(G - RING + decltype(s)::value, s, F{}); });

  // ---- epilogue: RoPE on the lane's dimension pairs (d and d + D/2 sit in the same lane), then the
  // dot with every query row slot (rows past RH are zero) in fp32; the two dimension halves of a
  // token combine with one shuffle
  float rlo[HALF_BLK][4][4], rhi[HALF_BLK][4][4];
#pragma unroll
  for (int rb = 0; rb < HALF_BLK; ++rb)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const float cv[4] = {cw[rb][v4].x, cw[rb][v4].y, cw[rb][v4].z, cw[rb][v4].w};
      const float sv[4] = {sw[rb][v4].x, sw[rb][v4].y, sw[rb][v4].z, sw[rb][v4].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float klo = acc[rb][v4 * 4 + e];
        const float khi = acc[rb + HALF_BLK][v4 * 4 + e];
        rlo[rb][v4][e] = klo * cv[e] - khi * sv[e];
        rhi[rb][v4][e] = khi * cv[e] + klo * sv[e];
      }
    }
  float xs[kSmallRows], mx[kSmallRows], sm[kSmallRows];
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) {
    float part = 0.0f;
#pragma unroll
    for (int rb = 0; rb < HALF_BLK; ++rb)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const int j = rb * 32 + 8 * v4 + 4 * lhi;  // pair index, 0 .. D/2-1
        const float4 qlo = *(const float4*)(q_s + r * D + j);
        const float4 qhi = *(const float4*)(q_s + r * D + j + HALF_D);
        part += qlo.x * rlo[rb][v4][0] + qlo.y * rlo[rb][v4][1] + qlo.z * rlo[rb][v4][2] + qlo.w * rlo[rb][v4][3] +
                qhi.x * rhi[rb][v4][0] + qhi.y * rhi[rb][v4][1] + qhi.z * rhi[rb][v4][2] + qhi.w * rhi[rb][v4][3];
      }
    const float full = sum_xor32(part);  // the lane's and its partner's dimension halves
    xs[r] = n < count ? full * a.scaling : -INFINITY;
  }
  // each wave's (max, sum exp) over its 32 tokens, then the workgroup's over its NW waves
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) mx[r] = max32(xs[r]);
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) sm[r] = mx[r] == -INFINITY ? 0.0f : sum32(__expf(xs[r] - mx[r]));
  if (lane == 0) {
    *(float4*)&stat_m[wave][0] = make_float4(mx[0], mx[1], mx[2], mx[3]);
    *(float4*)&stat_s[wave][0] = make_float4(sm[0], sm[1], sm[2], sm[3]);
  }
  static_assert(kSmallRows == 4, "statistics move as float4");
  __syncthreads();
  float4 wm[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) wm[w] = *(const float4*)&stat_m[w][0];
  float Mt[kSmallRows];
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, r == 0 ? wm[w].x : r == 1 ? wm[w].y : r == 2 ? wm[w].z : wm[w].w);
    Mt[r] = M;
  }
  // the workgroup's sum of exponentials per row, in wave 0: lane (w, r) = (lane / 4 % NW, lane % 4)
  // scales wave w's sum of row r to the maximum, and lane exchanges add the NW waves
  if (wave == 0) {
    const int w = (lane >> 2) % NW, r = lane & 3;
    const float M = r == 0 ? Mt[0] : r == 1 ? Mt[1] : r == 2 ? Mt[2] : Mt[3];
    const float mw = stat_m[w][r];
    float S = (M == -INFINITY || mw == -INFINITY) ? 0.0f : stat_s[w][r] * __expf(mw - M);
#pragma unroll
    for (int m = 4; m < 4 * NW; m <<= 1) S += __shfl_xor(S, m);
    if (lane < RH) {
      const long o = (long)(h * RH + lane) * a.nstats + tp;
      a.tile_max[o] = M;
      a.tile_sum[o] = S;
    }
  }
  // probabilities relative to the workgroup's maximum, fp16; every slot of its tokens is written (0
  // past the tile's tokens); the two lanes of a token write alternate rows
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r) {
    if (r >= RH) break;
    if ((r & 1) != lhi) continue;
    const float p = (xs[r] == -INFINITY) ? 0.0f : __expf(xs[r] - Mt[r]);
    a.probs[prob_index((long)h * RH + r, (long)tile * kTileTok + n, a.Hq * a.q_len)] = f16_bits(p);
  }
}

// ---------------------------------------------------------------------------
// Softmax statistics of the compressed part of sequence b, row `row`.
// ---------------------------------------------------------------------------
DKV_DEVICE int tiles_before(const int32_t* cu, int b, int tile) {
  int base = 0;
  for (int i = 0; i < b; ++i) base += (cu[i + 1] - cu[i] + tile - 1) / tile;
  return base;
}

// ---------------------------------------------------------------------------
// K3c: one workgroup per (sequence, output row).  It merges the tiles'
// softmax statistics of the compressed part with the exact tokens' (sinks,
// recent window, new tokens; computed beside K3b, row_exact) in one softmax
// and writes the row's output.
// ---------------------------------------------------------------------------
constexpr int kChunkLoads = 8;  // chunk partials per thread issued in the first round

// The exact tail of output row wg = b * R_total + row, in extra workgroups of K3b: the row's scores
// against its sequence's exact tokens (mask added), their maximum Me, Le = sum_e exp(s_e - Me) and
// ve[d] = sum_e exp(s_e - Me) v_e[d].  It needs only the query and the exact tokens, so it runs
// beside K3b's chunk workgroups (their registers and LDS leave room on every CU) instead of on the
// finish kernel's critical path.
//
// The exact tokens are cut into kExactParts contiguous shares, each taken by one wave of its own
// workgroup (the workgroups' loads then spread over kExactParts CUs): share `part` writes its
// (Me, Le, ve) to ex[wg * kExactParts + part], and the finish kernel merges the shares.  A wave's
// query, keys of its first kExactKR * 8 tokens and values of its first kExactVR * (256 / D) go
// out in one round (every load unconditional, with clamped indices: a load under a per-element
// condition is a branch and a wait each).  Scores: eight lanes
// per token, 8 tokens per round; lane ks holds the key's 16-byte pieces ks, ks + 8, ..., so each
// load of a round reads whole 128-byte lines; the dot products are reduced with three lane
// exchanges.  The weights go through the wave's own LDS area (a wave's LDS accesses run in order);
// values: a lane holds 4 consecutive dimensions of one token slot (D / 4 lanes per token), the
// slots combined with lane exchanges.
constexpr int kExactParts = 4;                        // token shares (workgroups) per output row
constexpr int kExactShare = kMaxExact / kExactParts;  // most tokens of one share
constexpr int kExactLds = 128 + kExactShare;          // floats: the query and the share's weights
constexpr int kExactKR = 2;  // key rounds (8 tokens each) loaded in the first round
constexpr int kExactKI = 4;  // key loads (16 bytes per lane) per round at D = 128 (2 at D = 64)
constexpr int kExactVR = 8;  // value loads (16 bytes per lane) in the first round

// Four consecutive elements (16 bytes of f32, 8 of f16 / bf16) of an exact key or value row as floats;
// the conversion from f16 / bf16 is exact, so every type gives the f32 path's results.
template <int XT>
DKV_DEVICE float4 load_exact4(const void* base, long e) {
  if constexpr (XT == DKV_F32) {
    return *(const float4*)((const float*)base + e);
  } else {
    const uint2 w = *(const uint2*)((const uint16_t*)base + e);
    if constexpr (XT == DKV_F16)
      return make_float4(half_bits_to_float((uint16_t)(w.x & 0xffffu)), half_bits_to_float((uint16_t)(w.x >> 16)),
                         half_bits_to_float((uint16_t)(w.y & 0xffffu)), half_bits_to_float((uint16_t)(w.y >> 16)));
    else
      return make_float4(bf16_bits_to_float((uint16_t)(w.x & 0xffffu)), bf16_bits_to_float((uint16_t)(w.x >> 16)),
                         bf16_bits_to_float((uint16_t)(w.y & 0xffffu)), bf16_bits_to_float((uint16_t)(w.y >> 16)));
  }
}

template <int XT>
__device__ void row_exact(const RowMergeArgs& a, int wg, int part, float* smem) {
  const int lane = threadIdx.x;
  if (lane >= 64) return;  // one wave
  float* q = smem;          // [128] the query row
  float* se = q + 128;      // [kExactShare] this share's scores, then weights
  const int row = wg % a.R_total;
  const int b = wg / a.R_total;
  const int D = a.D;
  const int gq = a.Hq / a.Hkv;
  const int qh = row / a.q_len, qi = row % a.q_len;
  const int h = qh / gq;
  const int e_seq = a.batch == 1 ? a.e0_single : a.cu_exact ? a.cu_exact[b] : 0;
  const int E_seq = a.batch == 1 ? a.e_single : a.cu_exact ? a.cu_exact[b + 1] - e_seq : 0;
  const int per = (E_seq + kExactParts - 1) / kExactParts;
  const int j0s = min(part * per, E_seq);  // this share: sequence-relative tokens j0s .. j0s + E - 1
  const int E = min(per, E_seq - j0s);
  const int e0 = e_seq + j0s;
  const long qbase = (((long)b * a.Hq + qh) * a.q_len + qi) * D;
  const uint32_t qw0 = load_query_word(a.query, qbase + min(lane, D - 1), a.query_dtype);
  const uint32_t qw1 = load_query_word(a.query, qbase + min(lane + 64, D - 1), a.query_dtype);
  // scores: lane (kj, ks) takes dimensions 4 ks + 32 i .. +4 (i < D / 32) of token kj of each round
  const int kj = lane >> 3, ks = lane & 7;
  const int ni = D / 32;
  const long krow0 = ((long)h * a.E_total + e0) * D + 4 * ks;  // element index
  const float* mrow0 = a.mask ? a.mask + (long)qi * E_seq + j0s : nullptr;
  // values: lane (tp, dq) holds dimensions 4 dq .. 4 dq + 3 of token slot tp
  const int lpt = D / 4;  // lanes per token
  const int tpi = 64 / lpt;  // tokens per value load
  const int dq = lane % lpt, tp = lane / lpt;
  const long vrow0 = ((long)h * a.E_total + e0) * D + 4 * dq;  // element index
  float4 k4[kExactKR][kExactKI];
  float mv[kExactKR];
  float4 v4[kExactVR];
  if (E > 0) {
#pragma unroll
    for (int r = 0; r < kExactKR; ++r) {
      const long kr = krow0 + (long)min(r * 8 + kj, E - 1) * D;
#pragma unroll
      for (int i = 0; i < kExactKI; ++i) k4[r][i] = load_exact4<XT>(a.key_exact, kr + 32 * min(i, ni - 1));
      mv[r] = mrow0 ? mrow0[min(r * 8 + kj, E - 1)] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kExactVR; ++i) v4[i] = load_exact4<XT>(a.value_exact, vrow0 + (long)min(tp + i * tpi, E - 1) * D);
  }
  if (lane < D) q[lane] = query_word_value(qw0, qbase + lane, a.query_dtype);
  if (lane + 64 < D) q[lane + 64] = query_word_value(qw1, qbase + lane + 64, a.query_dtype);
  float ex_m = -INFINITY, ex_l = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (E > 0) {
    float4 qv[kExactKI];  // this lane's query dimensions
#pragma unroll
    for (int i = 0; i < kExactKI; ++i) qv[i] = *(const float4*)(q + 4 * ks + 32 * min(i, ni - 1));
    auto score = [&](const float4 (&kk)[kExactKI], float mval, int j) {
      float dot = 0.0f;
#pragma unroll
      for (int i = 0; i < kExactKI; ++i) {
        const float d4 = qv[i].x * kk[i].x + qv[i].y * kk[i].y + qv[i].z * kk[i].z + qv[i].w * kk[i].w;
        dot += i < ni ? d4 : 0.0f;
      }
      dot = sum8(dot);
      const float sc = dot * a.scaling + mval;
      if (ks == 0 && j < E) se[j] = sc;
      return j < E ? sc : -INFINITY;
    };
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < kExactKR; ++r) m = fmaxf(m, score(k4[r], mv[r], r * 8 + kj));
    for (int j0 = kExactKR * 8; j0 < E; j0 += 8) {  // more than kExactKR * 8 tokens in the share
      float4 kk[kExactKI];
      const long kr = krow0 + (long)min(j0 + kj, E - 1) * D;
#pragma unroll
      for (int i = 0; i < kExactKI; ++i) kk[i] = load_exact4<XT>(a.key_exact, kr + 32 * min(i, ni - 1));
      const float mval = mrow0 ? mrow0[min(j0 + kj, E - 1)] : 0.0f;
      m = fmaxf(m, score(kk, mval, j0 + kj));
    }
    ex_m = wave_max(m);
    float l = 0.0f;
    for (int j = lane; j < E; j += 64) {
      const float s = se[j];
      const float w = (ex_m == -INFINITY || s == -INFINITY) ? 0.0f : __expf(s - ex_m);
      se[j] = w;
      l += w;
    }
    ex_l = wave_sum(l);
    // weighted values: every weight read is unconditional (clamped), the select drops the products
    // of slots past the share's tokens
#pragma unroll
    for (int i = 0; i < kExactVR; ++i) {
      const int t = tp + i * tpi;
      const float w = t < E ? se[min(t, kExactShare - 1)] : 0.0f;
      acc.x += w * v4[i].x;
      acc.y += w * v4[i].y;
      acc.z += w * v4[i].z;
      acc.w += w * v4[i].w;
    }
    for (int t0 = kExactVR * tpi; t0 < E; t0 += tpi) {  // tokens past the first round's values
      const int t = t0 + tp;
      const float4 vv = load_exact4<XT>(a.value_exact, vrow0 + (long)min(t, E - 1) * D);
      const float w = t < E ? se[min(t, kExactShare - 1)] : 0.0f;
      acc.x += w * vv.x;
      acc.y += w * vv.y;
      acc.z += w * vv.z;
      acc.w += w * vv.w;
    }
  }
  // the token slots' sums: lanes dq, dq + lpt, ... (D = 128: two slots; D = 64: four)
  if (lpt == 16) {
    acc.x = sum_xor16(acc.x);
    acc.y = sum_xor16(acc.y);
    acc.z = sum_xor16(acc.z);
    acc.w = sum_xor16(acc.w);
  }
  acc.x = sum_xor32(acc.x);
  acc.y = sum_xor32(acc.y);
  acc.z = sum_xor32(acc.z);
  acc.w = sum_xor32(acc.w);
  float* ex = a.ex + ((long)wg * kExactParts + part) * (D + 2);
  if (tp == 0) {  // ex + 2 + 4 dq is 8-byte aligned only
    ex[2 + 4 * dq] = acc.x;
    ex[3 + 4 * dq] = acc.y;
    ex[4 + 4 * dq] = acc.z;
    ex[5 + 4 * dq] = acc.w;
  }
  if (lane == 0) {
    ex[0] = ex_m;
    ex[1] = ex_l;
  }
}

// The finish kernel's work for one output row: merge the compressed part's tile statistics with the
// exact tail's (Me, Le) in one softmax and write the row's output
//   out = (e_c * (sum of the chunk partials) + e_c * L_c * mean_v + e_e * ve) / (e_c * L_c + e_e * L_e),
//   e_c = exp(M_c - M), e_e = exp(M_e - M), M = max(M_c, M_e).
// All its loads (tile statistics, the exact results, the chunk partials, the mean) go out in one round.
// PER_TILE: softmax-statistics entries per tile (1, or 2 for 128-token entries).
template <int NT, int PER_TILE>
__device__ void row_merge(const RowMergeArgs& a, int wg, float* smem) {
  float* bc = smem;      // [2] the compressed part's (max, sum)
  float* cbuf = bc + 2;  // [NT] per-thread chunk-partial sums
  const int row = wg % a.R_total;
  const int b = wg / a.R_total;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int D = a.D;
  const int gq = a.Hq / a.Hkv;
  const int qh = row / a.q_len, qi = row % a.q_len;
  const int h = qh / gq;
  const int d = tid % D, part = tid / D, parts = NT / D;
  // the sequence's statistics entries: PER_TILE per tile (an entry past its tokens holds (-inf, 0))
  constexpr int per_tile = PER_TILE;
  const int tb0 = tiles_before(a.cu_seqlens, b, kTileTok) * per_tile;
  const int2 sr = seq_range(a.cu_seqlens, a.batch, a.n_total, b);
  const int ntb = (sr.y - sr.x + kTileTok - 1) / kTileTok * per_tile;
  const float* tm = ntb > 0 ? a.tile_max + (long)row * a.nstats + tb0 : a.mean_v;
  const float* ts = ntb > 0 ? a.tile_sum + (long)row * a.nstats + tb0 : a.mean_v;
  float m4[4], s4[4];
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = min(lane + 64 * k, max(ntb - 1, 0));
      m4[k] = tm[t];
      s4[k] = ts[t];
    }
  }
  // the exact tail's shares (row_exact): (Me, Le) and ve[d] of each
  const float* ex = a.ex + (long)wg * kExactParts * (D + 2);
  float2 mlp[kExactParts];
  float vep[kExactParts];
#pragma unroll
  for (int p = 0; p < kExactParts; ++p) {
    mlp[p] = *(const float2*)(ex + p * (D + 2));
    vep[p] = ex[p * (D + 2) + 2 + d];
  }
  // thread (d, part) sums the chunk partials part, part + parts, ... of output d
  const long rows_all = (long)a.batch * a.R_total;
  const float* cp = a.out_part + (long)wg * D + d;
  float cv[kChunkLoads];
#pragma unroll
  for (int i = 0; i < kChunkLoads; ++i) cv[i] = cp[(long)min(part + i * parts, a.nchunks - 1) * rows_all * D];
  const float mv = a.mean_v[((long)a.layer * a.Hkv + h) * D + d];
  if (wave == 0) {  // the compressed part's online (max, sum) over this lane's tiles
    float mm = -INFINITY, ll = 0.0f;
    auto merge = [&](float mt, float st) {
      if (mt == -INFINITY) return;
      if (mt > mm) {
        ll = ll * __expf(mm - mt) + st;
        mm = mt;
      } else {
        ll += st * __expf(mt - mm);
      }
    };
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (lane + 64 * k < ntb) merge(m4[k], s4[k]);
    for (int t = lane + 256; t < ntb; t += 64) merge(tm[t], ts[t]);
    const float m = wave_max(mm);
    const float l = wave_sum(mm == -INFINITY ? 0.0f : ll * __expf(mm - m));
    if (lane == 0) {
      bc[0] = m;
      bc[1] = l;
    }
  }
  float cs = 0.0f;
#pragma unroll
  for (int i = 0; i < kChunkLoads; ++i) cs += part + i * parts < a.nchunks ? cv[i] : 0.0f;
  for (int c = part + kChunkLoads * parts; c < a.nchunks; c += parts) cs += cp[(long)c * rows_all * D];
  cbuf[tid] = cs;
  __syncthreads();
  if (tid < D) {
    float csum = 0.0f;
    for (int p = 0; p < parts; ++p) csum += cbuf[p * D + tid];
    float Me = -INFINITY, Le = 0.0f, ve = 0.0f;
#pragma unroll
    for (int p = 0; p < kExactParts; ++p) Me = fmaxf(Me, mlp[p].x);
#pragma unroll
    for (int p = 0; p < kExactParts; ++p) {
      const float f = mlp[p].x == -INFINITY ? 0.0f : __expf(mlp[p].x - Me);
      Le += mlp[p].y * f;
      ve += vep[p] * f;
    }
    const float Mc = bc[0], Lc = bc[1];
    const float M = fmaxf(Mc, Me);
    const float ec = (M == -INFINITY || Mc == -INFINITY) ? 0.0f : __expf(Mc - M);
    const float ee = (M == -INFINITY || Me == -INFINITY) ? 0.0f : __expf(Me - M);
    const float denom = ec * Lc + ee * Le;
    const float value = denom > 0.0f ? (ec * csum + ec * Lc * mv + ee * ve) / denom : 0.0f;
    store_from_float(a.out, (((long)b * a.q_len + qi) * a.Hq + qh) * D + tid, a.out_dtype, value);
  }
}


struct K3aArgs {
  const uint8_t* vcodes;  // decoded value codes, u8 [G][n_slots/16][64][16] (vcode_index)
  const float2* vaff;     // (scale, offset) per (group, token): value = code * scale + offset
  const int32_t* cu_seqlens;
  const uint16_t* probs;  // fp16 exp(score - tile max), [n_slots/16][R][16] (prob_index)
  const float* tile_max;
  float* w_part;
  // nstats: softmax-statistics entries per row (ntiles, or 2 * ntiles for 128-token entries)
  int batch, R_total, n_total, n_slots, nstats, G, rank, nsplits, row_blocks;
  int total_wg, per_xcd;  // workgroups, and consecutive workgroup indices per XCD
};

constexpr int kK3WaveTok = 128;  // tokens per K3a wave

// ---------------------------------------------------------------------------
// K1 for the value side: every token's value codes (all hot planes) as 8-bit
// codes, transposed to [G][n_slots/16][64][16] so that an MFMA operand (one
// component, 8 consecutive slots) is one 8-byte load and a wave's 32
// components of one 16-slot block are 512 contiguous bytes, plus the
// per-(group, slot) affine form (scale = span / 256, offset = low + span *
// 2^-(m+1); 0 and 0 for a group without planes or a padding slot).  One block
// = 256 slots x one group, one thread per slot, whose codes are one contiguous
// 16 KB run; the codes are transposed through LDS.
// ---------------------------------------------------------------------------
DKV_DEVICE void decode_values_block(const DecodeArgs& a, uint8_t* vcodes, float2* vaff, int2* tab, int id) {
  __shared__ uint32_t tile[64][kDecodeSlots / 4 + 1];  // [component][slot / 4], bytes of 4 slots per word
  const int nsb = a.n_slots / kDecodeSlots;
  const int2 bg = decode_block(a.G, nsb * a.G, id);
  const int sb = bg.x, g = bg.y;
  if (sb >= nsb) return;  // the whole block
  const int tl = threadIdx.x;
  const int slot = sb * kDecodeSlots + tl;
  const int t = slot_token(a, slot);
  const int row = t >= 0 ? a.s.pieces[t] : 0;
  const long toff = t >= 0 ? a.s.tok_off[t] : 0;
  stage_table_column(a.s, a.G, g, tab);
  __syncthreads();
  const SegmentWords sw = load_token_segment(a.s, tab, t, row, toff, 8);
  uint32_t cw[2][8];  // byte i of cw[h][w] is component 32h + 4w + i
  float2 aff;
  if (a.s.format == DKV_FMT_LADDER) {
    // value = code * scale + low: the affine pair is (scale, low)
#pragma unroll
    for (int h = 0; h < 2; ++h) ladder_segment_half(sw.w, sw.m, h, cw[h]);
    aff = make_float2(half_bits_to_float((uint16_t)(sw.header >> 16)),
                      half_bits_to_float((uint16_t)(sw.header & 0xffffu)));
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t pl[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) pl[q] = sw.w[2 * q + h];
      cw[h][0] = assemble_codes<0>(pl);
      cw[h][1] = assemble_codes<1>(pl);
      cw[h][2] = assemble_codes<2>(pl);
      cw[h][3] = assemble_codes<3>(pl);
      cw[h][4] = assemble_codes<4>(pl);
      cw[h][5] = assemble_codes<5>(pl);
      cw[h][6] = assemble_codes<6>(pl);
      cw[h][7] = assemble_codes<7>(pl);
    }
    const AffineDq dq = affine_from_header(sw.header, sw.m);
    aff = make_float2(dq.scale, dq.offset);
  }
  vaff[(long)g * a.n_slots + slot] = aff;
  uint8_t* tb8 = (uint8_t*)&tile[0][0];
  constexpr int ROWB = (kDecodeSlots / 4 + 1) * 4;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int w = 0; w < 8; ++w)
#pragma unroll
      for (int i = 0; i < 4; ++i) tb8[(h * 32 + 4 * w + i) * ROWB + tl] = (uint8_t)(cw[h][w] >> (8 * i));
  __syncthreads();
  // the block's 16 blocks of 16 slots x 64 components are 16 KB of contiguous codes; store j of
  // wave wv writes 16-slot block 4j + wv, component = lane: 1 KB of consecutive bytes per store
  const int wv = tl >> 6, c = tl & 63;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b16 = 4 * j + wv;
    const uint4 v = make_uint4(tile[c][b16 * 4], tile[c][b16 * 4 + 1], tile[c][b16 * 4 + 2], tile[c][b16 * 4 + 3]);
    *(uint4*)(vcodes + vcode_index(g, c, (long)sb * kDecodeSlots + b16 * 16, a.n_slots)) = v;
  }
}

// K1 as one launch: blocks [0, key_blocks) decode the keys, the rest (when a value stream is given)
// the values.  Not every block is resident at once, so the value blocks start as the key blocks
// drain and their segment reads overlap the key blocks' operand writes.  Block ids of each part
// keep the XCD pattern (key_blocks is a multiple of 8).
__global__ __launch_bounds__(kDecodeSlots) void decode_codes_kernel(DecodeArgs k, DecodeArgs v, uint8_t* vcodes,
                                                                    float2* vaff, int key_blocks) {
  extern __shared__ int2 tab[];
  if ((int)blockIdx.x < key_blocks)
    decode_keys_block(k, tab, blockIdx.x);
  else
    decode_values_block(v, vcodes, vaff, tab, blockIdx.x - key_blocks);
}

// 8 codes (bytes of lo, hi) -> 8 fp16 values equal to the codes.  (0x6400 | c)
// is the fp16 number 1024 + c; subtracting 1024 is exact.
DKV_DEVICE half8 codes_to_half8(uint32_t lo, uint32_t hi) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const uint32_t w0 = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);
  const uint32_t w1 = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);
  const uint32_t w2 = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);
  const uint32_t w3 = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);
  const half2_t bias = {(half_t)1024.0f, (half_t)1024.0f};
  half2_t h0, h1, h2, h3;
  __builtin_memcpy(&h0, &w0, 4);
  __builtin_memcpy(&h1, &w1, 4);
  __builtin_memcpy(&h2, &w2, 4);
  __builtin_memcpy(&h3, &w3, 4);
  h0 -= bias;
  h1 -= bias;
  h2 -= bias;
  h3 -= bias;
  half8 r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

// ---------------------------------------------------------------------------
// K3a: w[row][k] = sum_t p[row][t] * value[t][k] for one token split, one
// 64-component group and one block of 32 rows, with p = exp(s - M_row).
// value = code * scale + offset, so
//   w = sum_t (p * scale)[row][t] * code[t][k]  +  sum_t p[row][t] * offset[t]:
// the first term is a 32x32x16 fp16 MFMA with A = p * scale and B = the codes
// (exact in fp16), the second a per-row scalar.  Wave w of the 8 takes tokens
// w*128 .. +128 of the split in 16-token steps; the waves' sums meet in LDS.
// ---------------------------------------------------------------------------
// WAVES waves of 128 tokens: a split of 1024 tokens (8 waves) or, when 1024-token splits would leave
// CUs idle (small contexts), 512 (4 waves: twice the workgroups, each with half the loads).
// PER_TILE: softmax-statistics entries per tile (1, or 2 for 128-token entries).
template <int WAVES, int PER_TILE>
__global__ __launch_bounds__(WAVES * 64) void value_weights_kernel(K3aArgs a) {
  constexpr int SPLIT = WAVES * kK3WaveTok;
  __shared__ float red[WAVES][32][65];
  __shared__ float ored[WAVES][32];
  __shared__ float Mrow[32];
  // each wave's tokens: scale * 2^e as fp16 and the offset as fp32 (both 0 past the split's tokens),
  // and the wave's factor f = exp(tile max - row max) of each of the block's rows
  __shared__ __attribute__((aligned(16))) half_t sw[WAVES][kK3WaveTok];
  __shared__ __attribute__((aligned(16))) float sofs[WAVES][kK3WaveTok];
  __shared__ __attribute__((aligned(16))) float sf[WAVES][32];

  // consecutive workgroup indices on one XCD: the group workgroups of a split share its
  // probability rows, which that XCD's L2 then fetches once
  const int bid = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (bid >= a.total_wg) return;
  const int rbk = bid % a.row_blocks;
  const int g = (bid / a.row_blocks) % a.G;
  const int sp = bid / (a.row_blocks * a.G);
  const int2 bs = find_tile(a.cu_seqlens, a.batch, a.n_total, SPLIT, sp);
  const int b = bs.x;
  const int2 sr = seq_range(a.cu_seqlens, a.batch, a.n_total, b);
  const int tok0 = sr.x + bs.y * SPLIT;
  const int count = min(SPLIT, sr.y - tok0);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int tb0 = tiles_before(a.cu_seqlens, b, kTileTok);
  const long slot0 = (long)(tb0 + bs.y * (SPLIT / kTileTok)) * kTileTok;  // first slot of the split
  constexpr int per_tile = PER_TILE;
  const int sb0 = tb0 * per_tile;              // the sequence's first statistics entry
  const int wt0 = wave * kK3WaveTok;  // first token of this wave, relative to tok0
  const int my_row = rbk * 32 + l32;
  const bool row_ok = my_row < a.R_total;

  // every global load of the wave goes out first, unconditionally (clamped indices): the tile
  // maxima of the block's rows (small, so they return first and the row maxima are known while
  // the bulk is in flight), this wave's tile maximum, then the affine pairs of its 128 tokens
  // (one 16-byte load per lane, staged in LDS for the broadcast reads), its probability rows and
  // value codes for all 8 steps.
  const int ntb = (sr.y - sr.x + kTileTok - 1) / kTileTok * per_tile;  // the sequence's entries
  const int mrow = rbk * 32 + ((tid >> 3) & 31), msub = tid & 7;  // 8 lanes per row (waves 4-7 repeat 0-3)
  static_assert(WAVES >= 4, "the row maxima take 256 threads");
  const float* tmrow = a.tile_max + (long)min(mrow, a.R_total - 1) * a.nstats + sb0;
  float tmv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) tmv[i] = tmrow[min(msub + 8 * i, ntb - 1)];
  // this wave's 128 tokens lie in one statistics entry; its maximum for this lane's row (a wave
  // past the sequence's tokens reads a clamped entry and discards it)
  const int tile = min(sb0 + (bs.y * SPLIT + wt0) / (kTileTok / PER_TILE), a.nstats - 1);
  const float mt_raw = a.tile_max[(long)min(my_row, a.R_total - 1) * a.nstats + tile];
  const float2* aff = a.vaff + (long)g * a.n_slots + slot0;
  const float4 aff2 = *(const float4*)(aff + wt0 + 2 * lane);
  // step st covers slots slot0 + wt0 + 16 st .. +16 (one 16-slot block): the wave's probability
  // rows are 1 KB and each half of its code operand 512 B of contiguous memory
  const uint16_t* prow = a.probs + prob_index(row_ok ? my_row : 0, slot0 + wt0, a.R_total) + lhi * 8;
  const uint8_t* col0 = a.vcodes + vcode_index(g, l32, slot0 + wt0, a.n_slots) + lhi * 8;
  const uint8_t* col1 = col0 + 32 * 16;
  constexpr int STEPS = kK3WaveTok / 16;  // 8
  half8 pt[STEPS];
  uint2 c0[STEPS], c1[STEPS];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    pt[st] = *(const half8*)(prow + (long)st * a.R_total * 16);
    c0[st] = *(const uint2*)(col0 + st * 64 * 16);
    c1[st] = *(const uint2*)(col1 + st * 64 * 16);
  }
  __builtin_amdgcn_sched_barrier(0);
  const float mt = (row_ok && wt0 < count) ? mt_raw : -INFINITY;
  // Power-of-two operand scaling.  scale = span / 256 of a low-variance group (about 6e-5 at
  // rank 2048) puts p * scale among fp16's subnormals, which keep only a few significant bits.
  // p <= 1, so scaling the wave's scales by the 2^e that brings their maximum into [2^14, 2^15)
  // keeps every operand in fp16's normal range (or exactly 0); the fp32 sums are multiplied by
  // 2^-e before they leave the wave, which is exact.
  int sexp = 0;
  const int ta = wt0 + 2 * lane;  // the split-relative tokens of this lane's two affine pairs
  const float smax = wave_max(fmaxf(ta < count ? fabsf(aff2.x) : 0.0f, ta + 1 < count ? fabsf(aff2.z) : 0.0f));
  if (smax > 0.0f) {
    int ex;
    (void)frexpf(smax, &ex);  // smax = m * 2^ex, 0.5 <= m < 1
    sexp = min(max(15 - ex, -126), 126);
  }
  const float sup = ldexpf(1.0f, sexp), sdown = ldexpf(1.0f, -sexp);
  {
    const bool ok0 = ta < count, ok1 = ta + 1 < count;
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    const half2_t w2 = {ok0 ? (half_t)(aff2.x * sup) : (half_t)0.0f, ok1 ? (half_t)(aff2.z * sup) : (half_t)0.0f};
    *(half2_t*)&sw[wave][2 * lane] = w2;
    *(float2*)&sofs[wave][2 * lane] = make_float2(ok0 ? aff2.y : 0.0f, ok1 ? aff2.w : 0.0f);
  }
  {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, msub + 8 * i < ntb ? tmv[i] : -INFINITY);
    for (int t = msub + 64; t < ntb; t += 8) m = fmaxf(m, tmrow[t]);  // sequences of more than 64 tiles
    m = max8(m);
    if (tid < 256 && msub == 0) Mrow[tid >> 3] = mrow < a.R_total ? m : -INFINITY;
  }
  __syncthreads();
  const float my_M = Mrow[l32];

  floatx16 acc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[nb][v] = 0.0f;
  float osum = 0.0f;

  // K2 left p~ = exp(s - tile max) in fp16; the tile's factor f = exp(tile max - row max) turns
  // p~ into p = exp(s - row max).  The wave's tokens lie in one tile, so f is constant over them
  // and multiplies the wave's sums once, after the MFMAs: the A operand is p~ * (scale * 2^e), one
  // packed fp16 product per token pair.
  const float f = (mt == -INFINITY) ? 0.0f : __expf(mt - my_M);
  if (lhi == 0) sf[wave][l32] = f;
  // every load above stayed inside the slot buffers (they extend a whole split past the last
  // tile); slots past the split's tokens get p = 0 by selection, whatever they hold.  Only the
  // wave holding a split's last token has such slots among its own; it runs a masked copy of the
  // steps, and a wave entirely past them runs none.
  auto steps = [&](auto masked) {
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      __builtin_amdgcn_sched_barrier(0);  // one step's LDS reads at a time
      const half8 wv = *(const half8*)&sw[wave][st * 16 + lhi * 8];
      const float4 o0 = *(const float4*)&sofs[wave][st * 16 + lhi * 8];
      const float4 o1 = *(const float4*)&sofs[wave][st * 16 + lhi * 8 + 4];
      const float ofs[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
      half8 pv = pt[st];
      if constexpr (decltype(masked)::value) {
        const int t8 = wt0 + st * 16 + lhi * 8;  // this lane's 8 tokens: t8 .. t8+7 (split-relative)
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = t8 + e < count ? pv[e] : (half_t)0.0f;
      }
      const half8 pa = pv * wv;
#pragma unroll
      for (int e = 0; e < 8; ++e) osum += (float)pv[e] * ofs[e];
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, codes_to_half8(c0[st].x, c0[st].y), acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, codes_to_half8(c1[st].x, c1[st].y), acc[1], 0, 0, 0);
    }
  };
  if (wt0 + kK3WaveTok <= count)
    steps(std::false_type{});
  else if (wt0 < count)
    steps(std::true_type{});
  osum = sum_xor32(osum) * f;
  // acc[nb][v]: component nb*32 + l32, row 8*(v/4) + 4*lhi + (v&3); each row's f, and 2^-sexp, which
  // undoes the operand scaling (the wave wrote sf itself: its LDS accesses run in order)
  __builtin_amdgcn_wave_barrier();
  float fr[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 f4 = *(const float4*)&sf[wave][8 * i + 4 * lhi];
    fr[4 * i] = f4.x * sdown;
    fr[4 * i + 1] = f4.y * sdown;
    fr[4 * i + 2] = f4.z * sdown;
    fr[4 * i + 3] = f4.w * sdown;
  }
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int v = 0; v < 16; ++v) red[wave][8 * (v >> 2) + 4 * lhi + (v & 3)][nb * 32 + l32] = acc[nb][v] * fr[v];
  if (lhi == 0) ored[wave][l32] = osum;
  __syncthreads();
  for (int e = tid; e < 32 * 64; e += WAVES * 64) {
    const int r = e >> 6, k = e & 63;
    const int row = rbk * 32 + r;
    float s = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      s += red[w][r][k];
      o += ored[w][r];
    }
    if (row < a.R_total) a.w_part[((long)sp * a.R_total + row) * a.rank + g * 64 + k] = s + o;
  }
}

// ---------------------------------------------------------------------------
// K3b: one workgroup per (sequence, KV head, 128-component chunk, 64-dimension
// slice): sum the head's value partials over the sequence's splits, multiply
// once by the value-basis block [128 components][64 dimensions].  Thread
// (dp, part) holds dimension pair dp of the slice for components part * 16
// .. +16; the head's rows go in passes of NR (4 covers a decoding step's rows:
// GQA group x q_len <= 4).
// ---------------------------------------------------------------------------
struct K3bArgs {
  const int32_t* cu_seqlens;
  const float* w_part;
  const uint16_t* value_basis;
  float* out_part;
  int batch, n_total, layer, Hkv, Hq, q_len, D, rank, R_total, nchunks;
  int split_tok;   // tokens per K3a split
  int n_exact_wg;  // leading workgroups that compute a share of one output row's exact tail each (row_exact)
};

constexpr int kK3bParts = 8;                  // component parts of a chunk
constexpr int kK3bComp = kChunk / kK3bParts;  // 16 components per thread
constexpr int kK3bDims = 64;                  // dimensions per workgroup

// (at most two waves per SIMD: the exact-tail role's registers are not capped for occupancy)
template <int NR, int XT>
__global__ __launch_bounds__(kRowThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void basis_apply_kernel(K3bArgs a, RowMergeArgs ex) {
  if ((int)blockIdx.x < a.n_exact_wg) {  // share blockIdx.x % kExactParts of output row blockIdx.x / kExactParts
    __shared__ __attribute__((aligned(16))) float xsm[kExactLds];
    row_exact<XT>(ex, blockIdx.x / kExactParts, blockIdx.x % kExactParts, xsm);
    return;
  }
  __shared__ __attribute__((aligned(16))) float W[NR][kChunk];  // the pass's summed weights
  __shared__ float red[kK3bParts][NR][kK3bDims + 2];             // per-part outputs
  const int nds = a.D / kK3bDims;
  const int bid = blockIdx.x - a.n_exact_wg;
  const int ds = bid % nds;
  const int c = (bid / nds) % a.nchunks;
  const int h = (bid / (nds * a.nchunks)) % a.Hkv;
  const int b = bid / (nds * a.nchunks * a.Hkv);
  const int tid = threadIdx.x;
  const int RH = (a.Hq / a.Hkv) * a.q_len;
  const int sp0 = tiles_before(a.cu_seqlens, b, a.split_tok);
  const int2 sr = seq_range(a.cu_seqlens, a.batch, a.n_total, b);
  const int nsp = (sr.y - sr.x + a.split_tok - 1) / a.split_tok;
  const int D = a.D;
  const int npair = D / 2;
  const int dp = tid & 31, part = tid >> 5;
  // the basis block and the first pass's split partials go out in one round; thread (dp, part)
  // holds components part * 16 + ii of dimension pair ds * 32 + dp, one dword each
  const uint32_t* bv = (const uint32_t*)(a.value_basis + (((long)a.layer * a.Hkv + h) * a.rank + (long)c * kChunk +
                                                         part * kK3bComp) * D) + ds * (kK3bDims / 2) + dp;
  uint32_t bw[kK3bComp];
#pragma unroll
  for (int ii = 0; ii < kK3bComp; ++ii) bw[ii] = bv[(long)ii * npair];
  const long sp_stride4 = (long)a.R_total * a.rank / 4;  // split stride in float4 units
  const int rr = tid >> 5, k4 = tid & 31;                // the W element of this thread: row rr, components 4 k4 ..
  // one pass over rows r0 .. r0 + NR - 1 (the first pass is not inside the loop: hoisted out of a
  // loop, the basis conversions below would wait for the basis loads before the split loads go out)
  auto pass = [&](int r0) {
    const int nr = min(NR, RH - r0);
    // W[rr][4 k4 ..] = sum over the sequence's splits, in split order (16 loads per batch in flight)
    if (rr < nr) {
      const float4* src = (const float4*)(a.w_part + ((long)sp0 * a.R_total + (long)h * RH + r0 + rr) * a.rank +
                                          (long)c * kChunk) + k4;
      float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int s0 = 0; s0 < nsp; s0 += 16) {
        float4 v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = src[(long)min(s0 + k, nsp - 1) * sp_stride4];
#pragma unroll
        for (int k = 0; k < 16; ++k) {  // past the last split the (finite) repeat is added as exactly 0
          const float keep = s0 + k < nsp ? 1.0f : 0.0f;
          sum.x += v[k].x * keep;
          sum.y += v[k].y * keep;
          sum.z += v[k].z * keep;
          sum.w += v[k].w * keep;
        }
      }
      *(float4*)&W[rr][4 * k4] = sum;
    }
    __syncthreads();
    // rows nr .. NR - 1 of W hold stale values; their sums are computed and never stored
    float acc0[NR], acc1[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc0[r] = acc1[r] = 0.0f;
#pragma unroll
    for (int q = 0; q < kK3bComp / 4; ++q) {
      float4 w4[NR];
#pragma unroll
      for (int r = 0; r < NR; ++r) w4[r] = *(const float4*)&W[r][part * kK3bComp + 4 * q];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t bb = bw[4 * q + e];
        const float b0 = half_bits_to_float((uint16_t)(bb & 0xffffu));
        const float b1 = half_bits_to_float((uint16_t)(bb >> 16));
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const float wv = e == 0 ? w4[r].x : e == 1 ? w4[r].y : e == 2 ? w4[r].z : w4[r].w;
          acc0[r] += wv * b0;
          acc1[r] += wv * b1;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      red[part][r][2 * dp] = acc0[r];
      red[part][r][2 * dp + 1] = acc1[r];
    }
    __syncthreads();
    for (int e = tid; e < nr * kK3bDims; e += 256) {
      const int r = e / kK3bDims, dd = e % kK3bDims;
      float s = 0.0f;
#pragma unroll
      for (int p = 0; p < kK3bParts; ++p) s += red[p][r][dd];
      a.out_part[(((long)c * a.batch + b) * a.R_total + (long)h * RH + r0 + r) * D + ds * kK3bDims + dd] = s;
    }
  };
  pass(0);
  for (int r0 = NR; r0 < RH; r0 += NR) {
    __syncthreads();  // W and red are reused
    pass(r0);
  }
}

template <int PER_TILE>
__global__ __launch_bounds__(kRowThreads) void finish_kernel(RowMergeArgs a) {
  __shared__ float smem[2 + kRowThreads];
  row_merge<kRowThreads, PER_TILE>(a, blockIdx.x, smem);
}

// ---------------------------------------------------------------------------
// Workspace layout and argument checks.
// ---------------------------------------------------------------------------
struct Layout {
  int ntiles, nsplits, split_tok, R_total, nchunks, n_total, n_slots;
  int stat_tok, nstats;  // tokens per softmax-statistics entry (256, or 128 with K2's half-tile workgroups), entries per row
  size_t coef, vcodes, vaff, probs, tile_max, tile_sum, w_part, out_part, exact, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

constexpr int kCUs = 256;

// One KV head per K2 workgroup (keys_scores_head_kernel) for decodes whose 256-row workgroups
// would leave CUs idle: D / 256 as many rows per workgroup, 256 / D times the workgroups, each
// the same length, and no partial results to merge.
inline bool k2_head_form(const dkv_attend_args_t* a, int ntiles) {
  if ((a->q_heads / a->kv_heads) * a->q_len > kSmallRows) return false;
  if (a->rank % 256 != 0) return false;  // whole rings of four groups
  const long wg = (long)ntiles * (a->kv_heads / (256 / a->head_dim));
  return wg < kCUs;
}

// Tokens per one-head K2 workgroup: half a tile (four waves) when twice the workgroups still fit one
// wave of the CUs (short contexts: each workgroup's main loop is then half as long), else a tile.
// The softmax statistics follow: one entry per workgroup's tokens.
inline int k2_head_tokens(const dkv_attend_args_t* a, int ntiles) {
  return k2_head_form(a, ntiles) && 2L * ntiles * a->kv_heads <= kCUs ? kTileTok / 2 : kTileTok;
}

// Workspace: [decoded key coefficients][decoded value codes][value affine][probabilities][tile statistics]
// [split partials][chunk partials][exact-tail results].
// The decoded areas are indexed by token slot (256 per tile, see slot_token).
// `values` false: no value-decode areas (question scoring decodes and reads the keys alone), so
// every later area starts right after the key operands.
Layout make_layout(const dkv_attend_args_t* a, bool values = true) {
  Layout L{};
  L.ntiles = 0;
  L.R_total = a->q_heads * a->q_len;
  // K3a splits of 1024 tokens, or of 512 when 1024 would give fewer workgroups than CUs
  auto count_splits = [&](int tok) {
    int n = 0;
    for (int b = 0; b < a->batch; ++b) n += (a->cu_seqlens_host[b + 1] - a->cu_seqlens_host[b] + tok - 1) / tok;
    return n;
  };
  for (int b = 0; b < a->batch; ++b) L.ntiles += (a->cu_seqlens_host[b + 1] - a->cu_seqlens_host[b] + kTileTok - 1) / kTileTok;
  L.split_tok = kSplitTok;
  L.nsplits = count_splits(kSplitTok);
  if ((long)L.nsplits * (a->rank / 64) * ((L.R_total + 31) / 32) < kCUs) {
    L.split_tok = kSplitTok / 2;
    L.nsplits = count_splits(L.split_tok);
  }
  L.n_total = a->cu_seqlens_host[a->batch];
  L.n_slots = L.ntiles * kTileTok + kSplitTok;
  L.nchunks = a->rank / kChunk;
  L.stat_tok = k2_head_tokens(a, L.ntiles);
  L.nstats = L.ntiles * (kTileTok / L.stat_tok);
  size_t off = 0;
  L.coef = off;
  off += align256((size_t)L.n_slots * a->rank * 2);
  L.vcodes = off;
  if (values) off += align256((size_t)L.n_slots * a->rank);
  L.vaff = off;
  if (values) off += align256((size_t)L.n_slots * (a->rank / 64) * 8);
  L.probs = off;
  off += align256((size_t)L.R_total * L.n_slots * 2);
  L.tile_max = off;
  off += align256((size_t)L.R_total * L.nstats * 4);
  L.tile_sum = off;
  off += align256((size_t)L.R_total * L.nstats * 4);
  L.w_part = off;
  off += align256((size_t)L.nsplits * L.R_total * a->rank * 4);
  L.out_part = off;
  off += align256((size_t)L.nchunks * a->batch * L.R_total * a->head_dim * 4);
  L.exact = off;
  off += align256((size_t)a->batch * L.R_total * kExactParts * (a->head_dim + 2) * 4);
  L.total = off;
  return L;
}

int check_attend(const dkv_attend_args_t* a, const char* what) {
  DKV_REQUIRE(a, DKV_EINVAL, "%s: args is null", what);
  int rc = dkv::check_stream(&a->key, what);
  if (rc) return rc;
  DKV_REQUIRE(a->head_dim == 64 || a->head_dim == 128, DKV_ESHAPE, "%s: head_dim must be 64 or 128 (got %d)", what,
              a->head_dim);
  DKV_REQUIRE(a->rank > 0 && a->rank % 256 == 0 && a->rank == 64 * dkv::stream_groups(a->key), DKV_ESHAPE,
              "%s: rank %d must be a multiple of 256 and equal 64 * groups (%d)", what, a->rank,
              dkv::stream_groups(a->key));
  DKV_REQUIRE(a->kv_heads > 0 && a->q_heads % a->kv_heads == 0, DKV_ESHAPE, "%s: q_heads %d not a multiple of %d",
              what, a->q_heads, a->kv_heads);
  DKV_REQUIRE(a->kv_heads % (256 / a->head_dim) == 0, DKV_ESHAPE, "%s: kv_heads %d must be a multiple of %d", what,
              a->kv_heads, 256 / a->head_dim);
  DKV_REQUIRE(a->layer >= 0 && a->layer < a->layers, DKV_ESHAPE, "%s: layer %d out of range", what, a->layer);
  DKV_REQUIRE(a->batch >= 1 && a->q_len >= 1, DKV_ESHAPE, "%s: batch/q_len must be >= 1", what);
  DKV_REQUIRE(a->cu_seqlens && a->cu_seqlens_host && a->positions && a->key_basis && a->mean_k && a->rope_cos &&
                  a->rope_sin && a->query,
              DKV_EINVAL, "%s: null pointer in arguments", what);
  DKV_REQUIRE(a->query_dtype >= DKV_F32 && a->query_dtype <= DKV_BF16, DKV_EINVAL, "%s: bad query dtype", what);
  DKV_REQUIRE(a->rope_rows > 0, DKV_ESHAPE, "%s: rope_rows must be > 0 (got %d)", what, a->rope_rows);
  DKV_REQUIRE(a->cu_seqlens_host[0] == 0, DKV_ESHAPE, "%s: cu_seqlens[0] must be 0", what);
  for (int b = 0; b < a->batch; ++b)
    DKV_REQUIRE(a->cu_seqlens_host[b + 1] >= a->cu_seqlens_host[b], DKV_ESHAPE, "%s: cu_seqlens not monotone", what);
  return DKV_OK;
}

// The arguments of the exact tail (row_exact, extra K3b workgroups) and the merge (K3c): one
// workgroup per (sequence, output row).
RowMergeArgs row_merge_args(const dkv_attend_args_t* a, const Layout& L, char* ws, int E_total) {
  RowMergeArgs m{};
  m.cu_seqlens = a->cu_seqlens;
  m.cu_exact = a->cu_exact;
  m.tile_max = (const float*)(ws + L.tile_max);
  m.tile_sum = (const float*)(ws + L.tile_sum);
  m.nstats = L.nstats;
  m.mean_v = a->mean_v;
  m.key_exact = a->key_exact;
  m.value_exact = a->value_exact;
  m.mask = a->mask;
  m.query = a->query;
  m.out_part = (const float*)(ws + L.out_part);
  m.ex = (float*)(ws + L.exact);
  m.out = a->out;
  m.out_dtype = a->out_dtype;
  m.nchunks = L.nchunks;
  m.scaling = a->scaling;
  m.batch = a->batch;
  m.n_total = L.n_total;
  m.e0_single = 0;  // cu_exact[0] == 0 (check_exact)
  m.e_single = a->cu_exact ? a->cu_exact_host[1] - a->cu_exact_host[0] : 0;
  m.layer = a->layer;
  m.Hkv = a->kv_heads;
  m.Hq = a->q_heads;
  m.q_len = a->q_len;
  m.D = a->head_dim;
  m.R_total = L.R_total;
  m.E_total = E_total;
  m.query_dtype = a->query_dtype;
  return m;
}

// The exact tokens of a decode: offsets, pointers and the per-sequence limit; E_total gets their total.
int check_exact(const dkv_attend_args_t* a, int& E_total, const char* what) {
  DKV_REQUIRE(!a->mask || a->batch == 1, DKV_ESHAPE, "%s: mask is only supported for batch == 1", what);
  DKV_REQUIRE(!a->cu_exact || (a->key_exact && a->value_exact), DKV_EINVAL, "%s: exact keys/values missing", what);
  DKV_REQUIRE(a->exact_dtype == DKV_F32 || a->exact_dtype == DKV_F16 || a->exact_dtype == DKV_BF16, DKV_EINVAL,
              "%s: exact_dtype %d is not DKV_F32, DKV_F16 or DKV_BF16", what, a->exact_dtype);
  {  // row_exact reads four elements per load: 16 bytes of f32, 8 of f16 / bf16
    const uintptr_t align = a->exact_dtype == DKV_F32 ? 16 : 8;
    DKV_REQUIRE(!a->cu_exact || ((uintptr_t)a->key_exact % align == 0 && (uintptr_t)a->value_exact % align == 0),
                DKV_EINVAL, "%s: exact keys/values must be %d-byte aligned", what, (int)align);
  }
  E_total = 0;
  if (a->cu_exact) {
    DKV_REQUIRE(a->cu_exact_host, DKV_EINVAL, "%s: cu_exact needs cu_exact_host", what);
    DKV_REQUIRE(a->cu_exact_host[0] == 0, DKV_ESHAPE, "%s: cu_exact[0] must be 0", what);
    for (int b = 0; b < a->batch; ++b) {
      const int e = a->cu_exact_host[b + 1] - a->cu_exact_host[b];
      DKV_REQUIRE(e >= 0 && e <= kMaxExact, DKV_ESHAPE, "%s: %d exact tokens (max %d)", what, e, kMaxExact);
    }
    E_total = a->cu_exact_host[a->batch];
  }
  return DKV_OK;
}

// Decoding writes probabilities in the value side's layout (and may split the rank); question
// scoring writes them row-major for the importance kernel and never splits.
int launch_keys_scores(const dkv_attend_args_t* a, const Layout& L, char* ws, hipStream_t st, bool scoring = false,
                       float* sub_max = nullptr, float* sub_sum = nullptr, uint16_t* probs = nullptr) {
  if (L.ntiles == 0) return DKV_OK;
  K2Args k{};
  k.coef = (const uint16_t*)(ws + L.coef);
  k.n_slots = L.n_slots;
  k.cu_seqlens = a->cu_seqlens;
  k.positions = a->positions;
  k.key_basis = a->key_basis;
  k.mean_k = a->mean_k;
  k.rope_cos = a->rope_cos;
  k.rope_sin = a->rope_sin;
  k.rope_rows = a->rope_rows;
  k.query = a->query;
  k.probs = probs ? probs : (uint16_t*)(ws + L.probs);
  k.sub_max = sub_max;
  k.sub_sum = sub_sum;
  k.tile_max = (float*)(ws + L.tile_max);
  k.tile_sum = (float*)(ws + L.tile_sum);
  k.scaling = a->scaling;
  k.batch = a->batch;
  k.layer = a->layer;
  k.Hkv = a->kv_heads;
  k.Hq = a->q_heads;
  k.q_len = a->q_len;
  k.G = dkv::stream_groups(a->key);
  k.n_total = L.n_total;
  k.ntiles = L.ntiles;
  k.nstats = L.nstats;
  k.query_dtype = a->query_dtype;
  const int HPW = 256 / a->head_dim;
  k.total_wg = L.ntiles * (a->kv_heads / HPW);
  k.per_xcd = (k.total_wg + 7) / 8;
  const dim3 grid(8 * k.per_xcd);
  // decoding (at most kSmallRows query rows per KV head) and question scoring are separate
  // instantiations, so neither epilogue's registers weigh on the other's main loop
  const bool small = (a->q_heads / a->kv_heads) * a->q_len <= kSmallRows;
  if (!scoring && k2_head_form(a, L.ntiles)) {  // decoding, one KV head per workgroup
    const bool half = L.stat_tok < kTileTok;     // half a tile per workgroup (k2_head_tokens)
    k.total_wg = L.ntiles * (half ? 2 : 1) * a->kv_heads;
    k.per_xcd = (k.total_wg + 7) / 8;
    const dim3 hgrid(8 * k.per_xcd);
    if (a->head_dim == 128 && half)
      hipLaunchKernelGGL((keys_scores_head_kernel<128, 4>), hgrid, dim3(256), 0, st, k);
    else if (a->head_dim == 128)
      hipLaunchKernelGGL((keys_scores_head_kernel<128, 8>), hgrid, dim3(512), 0, st, k);
    else if (half)
      hipLaunchKernelGGL((keys_scores_head_kernel<64, 4>), hgrid, dim3(256), 0, st, k);
    else
      hipLaunchKernelGGL((keys_scores_head_kernel<64, 8>), hgrid, dim3(512), 0, st, k);
    return dkv::check_launch("keys_scores (one head per workgroup)");
  }
  // probabilities: the value side's blocked layout when decoding, row-major [R][ntiles * 256] for
  // question scoring (read by the importance kernel)
  if (a->head_dim == 128) {
    if (small && !scoring)
      hipLaunchKernelGGL((keys_scores_kernel<128, true>), grid, dim3(kK2Threads), 0, st, k);
    else if (small)
      hipLaunchKernelGGL((keys_scores_kernel<128, true, true>), grid, dim3(kK2Threads), 0, st, k);
    else if (!scoring)
      hipLaunchKernelGGL((keys_scores_kernel<128, false>), grid, dim3(kK2Threads), 0, st, k);
    else
      hipLaunchKernelGGL((keys_scores_kernel<128, false, true>), grid, dim3(kK2Threads), 0, st, k);
  } else {
    if (small && !scoring)
      hipLaunchKernelGGL((keys_scores_kernel<64, true>), grid, dim3(kK2Threads), 0, st, k);
    else if (small)
      hipLaunchKernelGGL((keys_scores_kernel<64, true, true>), grid, dim3(kK2Threads), 0, st, k);
    else if (!scoring)
      hipLaunchKernelGGL((keys_scores_kernel<64, false>), grid, dim3(kK2Threads), 0, st, k);
    else
      hipLaunchKernelGGL((keys_scores_kernel<64, false, true>), grid, dim3(kK2Threads), 0, st, k);
  }
  return dkv::check_launch("keys_scores");
}

}  // namespace

extern "C" size_t dkv_attend_workspace_bytes(const dkv_attend_args_t* a) {
  if (check_attend(a, "dkv_attend_workspace_bytes")) return 0;
  return make_layout(a).total;
}

extern "C" int dkv_attend_prepare(const dkv_attend_args_t* a, int32_t plane_cap, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  int rc = check_attend(a, "dkv_attend_prepare");
  if (rc) return rc;
  DKV_REQUIRE(plane_cap >= 0 && plane_cap <= 8, DKV_EINVAL, "dkv_attend_prepare: plane_cap %d not in 0..8",
              plane_cap);
  DKV_REQUIRE(a->key.format == DKV_FMT_PLANES || plane_cap == 8, DKV_EINVAL,
              "dkv_attend_prepare: a plane cap needs a bit-plane key stream (ladder streams have no planes)");
  // only the decoded areas at the head of the workspace are written (the value codes only with a
  // value stream), so an attend workspace, or a score workspace for the keys alone, will do
  const Layout L = make_layout(a, a->value.blob != nullptr);
  DKV_REQUIRE(workspace && workspace_bytes >= L.probs, DKV_EWORKSPACE,
              "dkv_attend_prepare: workspace %zu B < required %zu B", workspace_bytes, L.probs);
  DecodeArgs d{};
  d.s = a->key;
  d.cu_seqlens = a->cu_seqlens;
  d.coef = (uint16_t*)((char*)workspace + L.coef);
  d.batch = a->batch;
  d.n_total = L.n_total;
  d.ntiles = L.ntiles;
  d.n_slots = L.n_slots;
  d.G = dkv::stream_groups(a->key);
  d.plane_cap = plane_cap;
  const int key_rows = a->key.format == DKV_FMT_LADDER ? a->key.ladder.rungs : a->key.order.pieces + 1;
  DKV_REQUIRE(key_rows <= kMaxTableRows, DKV_ESHAPE, "dkv_attend_prepare: key stream table has %d rows (at most %d)",
              key_rows, kMaxTableRows);
  const int key_blocks = (int)(((long)d.G * (L.n_slots / kDecodeSlots) + 7) / 8 * 8);
  DecodeArgs v = d;
  int value_blocks = 0, rows = key_rows;
  if (a->value.blob) {
    rc = dkv::check_stream(&a->value, "dkv_attend_prepare");
    if (rc) return rc;
    DKV_REQUIRE(dkv::stream_groups(a->value) == dkv::stream_groups(a->key), DKV_ESHAPE,
                "dkv_attend_prepare: K/V group mismatch");
    const int value_rows = a->value.format == DKV_FMT_LADDER ? a->value.ladder.rungs : a->value.order.pieces + 1;
    DKV_REQUIRE(value_rows <= kMaxTableRows, DKV_ESHAPE,
                "dkv_attend_prepare: value stream table has %d rows (at most %d)", value_rows, kMaxTableRows);
    v.s = a->value;
    v.plane_cap = 8;
    value_blocks = key_blocks;
    rows = std::max(rows, value_rows);
  }
  hipLaunchKernelGGL(decode_codes_kernel, dim3((unsigned)(key_blocks + value_blocks)), dim3(kDecodeSlots),
                     rows * sizeof(int2), dkv::as_stream(stream), d, v, (uint8_t*)((char*)workspace + L.vcodes),
                     (float2*)((char*)workspace + L.vaff), key_blocks);
  return dkv::check_launch("decode_codes");
}

static int check_values(const dkv_attend_args_t* a, int& E_total) {
  int rc = dkv::check_stream(&a->value, "dkv_attend_values");
  if (rc) return rc;
  DKV_REQUIRE(dkv::stream_groups(a->value) == dkv::stream_groups(a->key), DKV_ESHAPE,
              "dkv_attend_values: K/V group mismatch");
  DKV_REQUIRE(a->value_basis && a->mean_v && a->out, DKV_EINVAL, "dkv_attend_values: null value/out pointer");
  DKV_REQUIRE(a->out_dtype >= DKV_F32 && a->out_dtype <= DKV_BF16, DKV_EINVAL, "dkv_attend_values: bad out dtype");
  return check_exact(a, E_total, "dkv_attend_values");
}

extern "C" int dkv_attend_scores(const dkv_attend_args_t* a, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_attend(a, "dkv_attend_scores");
  if (rc) return rc;
  const Layout L = make_layout(a);
  DKV_REQUIRE(workspace && workspace_bytes >= L.total, DKV_EWORKSPACE,
              "dkv_attend_scores: workspace %zu B < required %zu B", workspace_bytes, L.total);
  return launch_keys_scores(a, L, (char*)workspace, dkv::as_stream(stream));
}

extern "C" int dkv_attend_values(const dkv_attend_args_t* a, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_attend(a, "dkv_attend_values");
  if (rc) return rc;
  int E_total = 0;
  rc = check_values(a, E_total);
  if (rc) return rc;
  const Layout L = make_layout(a);
  DKV_REQUIRE(workspace && workspace_bytes >= L.total, DKV_EWORKSPACE,
              "dkv_attend_values: workspace %zu B < required %zu B", workspace_bytes, L.total);
  char* ws = (char*)workspace;
  hipStream_t st = dkv::as_stream(stream);
  const int G = dkv::stream_groups(a->key);
  if (L.nsplits > 0) {  // K3a: one workgroup per (split, group, row block)
    K3aArgs k{};
    k.vcodes = (const uint8_t*)(ws + L.vcodes);
    k.vaff = (const float2*)(ws + L.vaff);
    k.cu_seqlens = a->cu_seqlens;
    k.probs = (const uint16_t*)(ws + L.probs);
    k.tile_max = (const float*)(ws + L.tile_max);
    k.w_part = (float*)(ws + L.w_part);
    k.batch = a->batch;
    k.R_total = L.R_total;
    k.n_total = L.n_total;
    k.n_slots = L.n_slots;
    k.nstats = L.nstats;
    k.G = G;
    k.rank = a->rank;
    k.nsplits = L.nsplits;
    k.row_blocks = (L.R_total + 31) / 32;
    k.total_wg = L.nsplits * k.row_blocks * G;
    k.per_xcd = (k.total_wg + 7) / 8;
    constexpr int W8 = kSplitTok / kK3WaveTok, W4 = kSplitTok / 2 / kK3WaveTok;
    const dim3 grid(8u * (unsigned)k.per_xcd);
    const bool whole = L.stat_tok == kTileTok;  // one statistics entry per tile
    if (L.split_tok == kSplitTok && whole)
      hipLaunchKernelGGL((value_weights_kernel<W8, 1>), grid, dim3(W8 * 64), 0, st, k);
    else if (L.split_tok == kSplitTok)
      hipLaunchKernelGGL((value_weights_kernel<W8, 2>), grid, dim3(W8 * 64), 0, st, k);
    else if (whole)
      hipLaunchKernelGGL((value_weights_kernel<W4, 1>), grid, dim3(W4 * 64), 0, st, k);
    else
      hipLaunchKernelGGL((value_weights_kernel<W4, 2>), grid, dim3(W4 * 64), 0, st, k);
    rc = dkv::check_launch("value_weights");
    if (rc) return rc;
  }
  // the exact tail (extra K3b workgroups) and the merge (K3c), one workgroup per (sequence, output row)
  const RowMergeArgs m = row_merge_args(a, L, ws, E_total);
  K3bArgs kb{};
  kb.cu_seqlens = a->cu_seqlens;
  kb.w_part = (const float*)(ws + L.w_part);
  kb.value_basis = a->value_basis;
  kb.out_part = (float*)(ws + L.out_part);
  kb.batch = a->batch;
  kb.n_total = L.n_total;
  kb.layer = a->layer;
  kb.Hkv = a->kv_heads;
  kb.Hq = a->q_heads;
  kb.q_len = a->q_len;
  kb.D = a->head_dim;
  kb.rank = a->rank;
  kb.R_total = L.R_total;
  kb.nchunks = L.nchunks;
  kb.split_tok = L.split_tok;
  kb.n_exact_wg = a->batch * L.R_total * kExactParts;
  const long k3b_blocks = kb.n_exact_wg + (long)a->batch * a->kv_heads * L.nchunks * (a->head_dim / kK3bDims);
  const bool rows4 = (a->q_heads / a->kv_heads) * a->q_len <= 4;
  auto k3b = [&](auto nr, auto xt) {
    hipLaunchKernelGGL((basis_apply_kernel<decltype(nr)::value, decltype(xt)::value>), dim3((unsigned)k3b_blocks),
                       dim3(kRowThreads), 0, st, kb, m);
  };
  using R4 = std::integral_constant<int, 4>;
  using R8 = std::integral_constant<int, 8>;
  using X32 = std::integral_constant<int, DKV_F32>;
  using X16 = std::integral_constant<int, DKV_F16>;
  using XB16 = std::integral_constant<int, DKV_BF16>;
  if (a->exact_dtype == DKV_F16) {
    if (rows4) k3b(R4{}, X16{}); else k3b(R8{}, X16{});
  } else if (a->exact_dtype == DKV_BF16) {
    if (rows4) k3b(R4{}, XB16{}); else k3b(R8{}, XB16{});
  } else {
    if (rows4) k3b(R4{}, X32{}); else k3b(R8{}, X32{});
  }
  rc = dkv::check_launch("basis_apply");
  if (rc) return rc;
  // K3c
  if (L.stat_tok == kTileTok)
    hipLaunchKernelGGL(finish_kernel<1>, dim3((unsigned)((long)a->batch * L.R_total)), dim3(kRowThreads), 0, st, m);
  else
    hipLaunchKernelGGL(finish_kernel<2>, dim3((unsigned)((long)a->batch * L.R_total)), dim3(kRowThreads), 0, st, m);
  return dkv::check_launch("finish");
}

extern "C" int dkv_attend_layer(const dkv_attend_args_t* a, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_attend(a, "dkv_attend_layer");
  if (rc) return rc;
  int E_total = 0;
  rc = check_values(a, E_total);
  if (rc) return rc;
  rc = dkv_attend_scores(a, workspace, workspace_bytes, stream);
  if (rc) return rc;
  return dkv_attend_values(a, workspace, workspace_bytes, stream);
}

// ===========================================================================
// K4a: question scoring of the hot tier (scripts/progressive.py:239-254 with
// scripts/dimmer.py:52-66).  Per layer: K2 scores every (query head, query
// position) row against the compressed keys and writes fp16 probabilities
// relative to the maximum of each 64-token tile quarter (row-major) with the
// quarters' softmax statistics; row_stats merges those statistics with the
// exact context tokens and the question's own keys (causal) into the row's
// maximum M and sum L; importance adds, to every token, the sum over rows of
// probability * exp(quarter max - M) / L, in a fixed order, so results do not
// depend on scheduling.
// ===========================================================================
namespace {

struct RowStatsArgs {
  const void* query;
  const float* key_exact;     // [Hkv][E][D]
  const float* key_question;  // [Hkv][Lq][D]
  const float* sub_max;       // [R_total][nsub] (compressed part per 64-token tile quarter, from K2)
  const float* sub_sum;
  float* stat;                // [R_total][2]: softmax maximum M and 1 / L over every key of the row
  float scaling;
  int Hkv, Hq, q_len, E, query_dtype, nsub;
};

// One workgroup (wg) per RPW consecutive rows of one query head (RPW divides q_len): the softmax
// statistics of each row over the compressed tokens (merged from K2's per-quarter maxima and sums),
// the exact context tokens and the question's own keys up to the row's position (causal).  The
// rows share their KV head, so each exact key is loaded once for all of them.  Every global load
// of the first round (the rows' quarter statistics, their query rows, the first pass of exact keys)
// is unconditional and goes out before any is used.  A pass scores 128 keys: the KL = NT / 128
// consecutive lanes KL k .. KL k + KL - 1 score key k, each over 1 / KL of the head dimension.
template <int D, int RPW, int NT>
DKV_DEVICE void row_stats_rows(const RowStatsArgs& a, int wg) {
  constexpr int kStatThreads = NT;
  constexpr int kStatWaves = NT / 64;
  constexpr int KL = NT / 128;                         // lanes per key (2 or 4)
  static_assert(KL == 2 || KL == 4, "lanes per key");
  constexpr int kStatKeys = NT / KL;                   // exact keys scored per pass
  constexpr int U = D / (4 * KL);                      // float4 per lane: 1 / KL of a key row
  constexpr int QW = (RPW * D + kStatThreads - 1) / kStatThreads;  // query elements per thread
  __shared__ __attribute__((aligned(16))) float q[RPW][D];
  __shared__ float red[2][kStatWaves][RPW];
  const int row0 = wg * RPW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kj = tid / KL, kh = tid % KL;
  const int gq = a.Hq / a.Hkv;
  const int qh = row0 / a.q_len, qi0 = row0 % a.q_len;
  const int h = qh / gq;
  const int nkeys_max = a.E + qi0 + RPW;  // row i sees exact context tokens + question keys 0..qi0 + i
  // lane kh of a key holds its 16-byte pieces kh, kh + KL, ...: the KL lanes of a key read one
  // contiguous run per load instead of one cache line each
  auto key_half = [&](int j) {
    return (const float4*)(j < a.E ? a.key_exact + ((long)h * a.E + j) * D
                                   : a.key_question + ((long)h * a.q_len + (j - a.E)) * D) + kh;
  };
  // first round: quarter statistics (one per row and thread), query words, the first pass of keys
  float mt[RPW], st[RPW];
  // the RPW rows' statistics of quarter t (eight rows of one block: 32 contiguous bytes per array)
  auto load_quarter = [&](int t) {
    if constexpr (RPW == 8) {
      const float4* pm = (const float4*)(a.sub_max + sub_index(row0, t, a.nsub));
      const float4* ps = (const float4*)(a.sub_sum + sub_index(row0, t, a.nsub));
      const float4 m0 = pm[0], m1 = pm[1], s0 = ps[0], s1 = ps[1];
      mt[0] = m0.x; mt[1] = m0.y; mt[2] = m0.z; mt[3] = m0.w; mt[4] = m1.x; mt[5] = m1.y; mt[6] = m1.z; mt[7] = m1.w;
      st[0] = s0.x; st[1] = s0.y; st[2] = s0.z; st[3] = s0.w; st[4] = s1.x; st[5] = s1.y; st[6] = s1.z; st[7] = s1.w;
    } else {
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        mt[i] = a.sub_max[sub_index(row0 + i, t, a.nsub)];
        st[i] = a.sub_sum[sub_index(row0 + i, t, a.nsub)];
      }
    }
  };
  load_quarter(max(min(tid, a.nsub - 1), 0));  // nsub = 0 (no compressed tokens): values nobody uses
  uint32_t qword[QW];
  const long qbase = ((long)qh * a.q_len + qi0) * D;  // the RPW rows' queries are contiguous
#pragma unroll
  for (int w = 0; w < QW; ++w) qword[w] = load_query_word(a.query, qbase + min(tid + w * kStatThreads, RPW * D - 1),
                                                          a.query_dtype);
  float4 k4[U];
  {
    const float4* kr = key_half(min(kj, nkeys_max - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) k4[u] = kr[u * KL];
  }
  __builtin_amdgcn_sched_barrier(0);
  // compressed part: the thread's quarters of each row
  float mc[RPW], lc[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const bool live = tid < a.nsub && mt[i] != -INFINITY;
    mc[i] = live ? mt[i] : -INFINITY;
    lc[i] = live ? st[i] : 0.0f;
  }
  for (int t0 = kStatThreads; t0 < a.nsub; t0 += kStatThreads) {  // more quarters than threads
    load_quarter(min(t0 + tid, a.nsub - 1));
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      if (t0 + tid >= a.nsub || mt[i] == -INFINITY) continue;
      if (mt[i] > mc[i]) {
        lc[i] = (mc[i] == -INFINITY ? 0.0f : lc[i] * __expf(mc[i] - mt[i])) + st[i];
        mc[i] = mt[i];
      } else {
        lc[i] += st[i] * __expf(mt[i] - mc[i]);
      }
    }
  }
#pragma unroll
  for (int w = 0; w < QW; ++w) {
    const int e = tid + w * kStatThreads;
    if (e < RPW * D) (&q[0][0])[e] = query_word_value(qword[w], qbase + e, a.query_dtype);
  }
  __syncthreads();
  // scores of the thread's key (both lanes of the pair get the full dot) for every row, RG rows at a
  // time (the scheduling barrier keeps the compiler from holding every row's query in registers)
  constexpr int RG = 256 / D;
  auto scores = [&](float (&sc)[RPW]) {
#pragma unroll
    for (int i0 = 0; i0 < RPW; i0 += RG) {
#pragma unroll
      for (int i = i0; i < i0 + RG && i < RPW; ++i) {
        float dot = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float4 q4 = *(const float4*)&q[i][4 * (kh + KL * u)];
          dot += q4.x * k4[u].x + q4.y * k4[u].y + q4.z * k4[u].z + q4.w * k4[u].w;
        }
        dot += lane_xor1(dot);  // the key's KL lanes (each sum is the same in all of them)
        if constexpr (KL == 4) dot += lane_xor2(dot);
        sc[i] = dot * a.scaling;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  float first[RPW], m[RPW];
  scores(first);
#pragma unroll
  for (int i = 0; i < RPW; ++i) m[i] = fmaxf(mc[i], kj < a.E + qi0 + i + 1 ? first[i] : -INFINITY);
  for (int j0 = kStatKeys; j0 < nkeys_max; j0 += kStatKeys) {  // more exact keys than one pass holds
    const float4* kr = key_half(min(j0 + kj, nkeys_max - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) k4[u] = kr[u * KL];
    float sc[RPW];
    scores(sc);
#pragma unroll
    for (int i = 0; i < RPW; ++i) m[i] = j0 + kj < a.E + qi0 + i + 1 ? fmaxf(m[i], sc[i]) : m[i];
  }
  // joint maxima, then the sums of exponentials (each key counted by its even lane)
#pragma unroll
  for (int i = 0; i < RPW; ++i) m[i] = wave_max(m[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) red[0][wave][i] = m[i];
  }
  __syncthreads();
  float M[RPW], l[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    M[i] = red[0][0][i];
#pragma unroll
    for (int w = 1; w < kStatWaves; ++w) M[i] = fmaxf(M[i], red[0][w][i]);
    l[i] = (mc[i] == -INFINITY || M[i] == -INFINITY) ? 0.0f : lc[i] * __expf(mc[i] - M[i]);
    l[i] += kh == 0 && kj < a.E + qi0 + i + 1 ? __expf(first[i] - M[i]) : 0.0f;
  }
  for (int j0 = kStatKeys; j0 < nkeys_max; j0 += kStatKeys) {
    const float4* kr = key_half(min(j0 + kj, nkeys_max - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) k4[u] = kr[u * KL];
    float sc[RPW];
    scores(sc);
#pragma unroll
    for (int i = 0; i < RPW; ++i) l[i] += kh == 0 && j0 + kj < a.E + qi0 + i + 1 ? __expf(sc[i] - M[i]) : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) l[i] = wave_sum(l[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) red[1][wave][i] = l[i];
  }
  __syncthreads();
  if (tid < RPW) {  // thread i writes row i: its maximum from the first exchange, its sum from the second
    float Mi = red[0][0][tid], L = 0.0f;
#pragma unroll
    for (int w = 0; w < kStatWaves; ++w) {
      Mi = fmaxf(Mi, red[0][w][tid]);
      L += red[1][w][tid];
    }
    a.stat[2 * (row0 + tid)] = Mi;
    a.stat[2 * (row0 + tid) + 1] = L > 0.0f ? 1.0f / L : 0.0f;
  }
}

// importance[t] += sum over rows r of p = exp(s - M_r) / L_r = probs[r][t] * exp(quarter max - M_r)
// / L_r: one workgroup per 64-token tile quarter.  Lane (row lane rl = lane / 8, token chunk
// tc = lane % 8) of wave w reads 8 tokens (16 B) of rows w * 8 + rl, + 64, + 128, ...; the row
// lanes, then the waves, are summed in a fixed order, so the result does not depend on scheduling.
struct ImportanceArgs {
  const uint16_t* probs;  // fp16 [R_total][ntiles * 256], relative to each quarter's maximum (K2)
  const float* sub_max;   // [R_total][ntiles * 4] quarter maxima (K2)
  const float* stat;      // [R_total][2]: M and 1 / L (row_stats_rows)
  float* importance;      // [n]
  int R_total, n, ntiles;
};

constexpr int kImpThreads = 512;
constexpr int kImpWaves = kImpThreads / 64;
constexpr int kImpBatch = 12;  // row iterations whose loads go out together

// sub: the tile quarter (tile sub / 4, quarter sub % 4)
DKV_DEVICE void importance_quarter(const ImportanceArgs& a, int sub) {
  __shared__ float part[kImpWaves][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rl = lane >> 3, tc = lane & 7;
  const long pos = (long)sub * 64 + tc * 8;
  const long pstride = (long)a.ntiles * kTileTok;
  const int nsub = a.ntiles * 4;
  constexpr int kRowStep = kImpWaves * 8;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int r0 = wave * 8 + rl; r0 < a.R_total; r0 += kRowStep * kImpBatch) {
    uint4 pv[kImpBatch];
    float mq[kImpBatch];
    float2 ml[kImpBatch];
#pragma unroll
    for (int k = 0; k < kImpBatch; ++k) {  // clamped rows: every load is unconditional
      const int r = min(r0 + kRowStep * k, a.R_total - 1);
      pv[k] = *(const uint4*)(a.probs + (long)r * pstride + pos);
      mq[k] = a.sub_max[sub_index(r, sub, nsub)];
      ml[k] = *(const float2*)(a.stat + 2 * r);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch goes out before the first is used
#pragma unroll
    for (int k = 0; k < kImpBatch; ++k) {
      const bool live = r0 + kRowStep * k < a.R_total && mq[k] != -INFINITY && ml[k].x != -INFINITY;
      const float f = live ? __expf(mq[k] - ml[k].x) * ml[k].y : 0.0f;
      const uint32_t w[4] = {pv[k].x, pv[k].y, pv[k].z, pv[k].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += half_bits_to_float((uint16_t)(w[i] & 0xffffu)) * f;
        acc[2 * i + 1] += half_bits_to_float((uint16_t)(w[i] >> 16)) * f;
      }
    }
  }
  // sum the 8 row lanes (lane bits 3..5) of each token chunk, then the waves
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float v = acc[i];
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    acc[i] = v;
  }
  if (rl == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) part[wave][tc * 8 + i] = acc[i];
  }
  __syncthreads();
  if (tid < 64) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kImpWaves; ++w) sum += part[w][tid];
    const int t = sub * 64 + tid;  // one sequence: token slots are tokens
    if (t < a.n) a.importance[t] += sum;
  }
}

// K4a per layer after K2: this layer's row statistics (the first n_stat_wg workgroups) beside the
// previous layer's importance (the others, one per tile quarter), whose probabilities, quarter
// maxima and row statistics sit in the other half of their double buffers.  The statistics are a
// chain of dependent loads on few workgroups and the importance a stream over the probabilities,
// so one launch overlaps them.  Layers are added to the importance in order, one launch late.
// (registers capped for two workgroups per CU: both roles then run beside each other on every CU)
template <int D, int RPW>
__global__ __launch_bounds__(kImpThreads) __attribute__((amdgpu_waves_per_eu(4)))
void score_stats_kernel(RowStatsArgs rs, ImportanceArgs im, int n_stat_wg) {
  if ((int)blockIdx.x < n_stat_wg)
    row_stats_rows<D, RPW, kImpThreads>(rs, blockIdx.x);
  else
    importance_quarter(im, blockIdx.x - n_stat_wg);
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// Probabilities, quarter maxima and row statistics are double-buffered by layer parity: the
// importance of layer l - 1 is computed while layer l's statistics are.
struct ScoreLayout {
  Layout base;
  size_t probs2, sub_max[2], sub_sum, stat[2], total;
};

// The attend layout without the value areas up to the tile statistics (decoded keys,
// probabilities), then the second probability buffer, the per-quarter statistics and the per-row
// statistics.
ScoreLayout make_score_layout(const dkv_attend_args_t* a) {
  ScoreLayout S{};
  S.base = make_layout(a, /*values=*/false);
  const size_t per_quarter = align256((size_t)((S.base.R_total + 7) / 8 * 8) * S.base.ntiles * 4 * 4);
  const size_t per_stat = align256((size_t)S.base.R_total * 2 * 4);
  size_t off = S.base.w_part;
  S.probs2 = off;
  off += align256((size_t)S.base.R_total * S.base.n_slots * 2);
  for (int i = 0; i < 2; ++i) {
    S.sub_max[i] = off;
    off += per_quarter;
  }
  S.sub_sum = off;
  off += per_quarter;
  for (int i = 0; i < 2; ++i) {
    S.stat[i] = off;
    off += per_stat;
  }
  S.total = off;
  return S;
}

// ---------------------------------------------------------------------------
// K4b: top-k by radix select in one workgroup (1024 threads).
// ---------------------------------------------------------------------------
constexpr int kTopkThreads = 1024;

DKV_DEVICE uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kTopkCache = 32;  // elements per thread kept in registers (n <= 32,768); larger n reloads

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ s, int n, int k,
                                                            int32_t* __restrict__ out) {
  constexpr int kWaves = kTopkThreads / 64;
  __shared__ uint32_t hist[kWaves][256];  // one histogram per wave: fewer LDS atomic collisions
  __shared__ uint32_t total[256];
  __shared__ uint32_t sh_prefix, sh_k;
  __shared__ uint32_t wmin[kWaves], wmax[kWaves];
  __shared__ int wsum_g[kWaves], wsum_e[kWaves];
  // the keys of thread t's range at kbuf[t * ps ..], ps = per rounded up to odd (conflict-free reads)
  __shared__ uint32_t kbuf[kTopkThreads * (kTopkCache + 1)];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (n + kTopkThreads - 1) / kTopkThreads;
  const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
  const bool cached = per <= kTopkCache;
  uint32_t key[kTopkCache];
  if (cached) {
    // coalesced loads into LDS, then each thread's contiguous range into registers; element e
    // belongs to thread e / per (computed in fp32: e < 2^15 and per <= 32 keep it exact)
    const int ps = per | 1;
    const float inv_per = 1.0f / (float)per;
    for (int e = tid; e < n; e += kTopkThreads) {
      const int q = (int)(((float)e + 0.5f) * inv_per);
      kbuf[q * ps + (e - q * per)] = order_key(s[e]);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTopkCache; ++j) key[j] = kbuf[tid * ps + min(j, per - 1)];
  }
  auto key_at = [&](int j) { return cached ? key[j] : order_key(s[i0 + j]); };
  // The keys' range [kmin, kmax]: the select runs on v = (key - kmin) << lz, which puts the range's
  // top bit at bit 31, so the first 8-bit digit already spreads the keys over the buckets (raw
  // float keys of similar magnitude share their top byte, and LDS atomics on one bucket serialize).
  uint32_t lo = 0xffffffffu, hi = 0u;
  for (int i = i0; i < i1; ++i) {
    const uint32_t u = key_at(i - i0);
    lo = min(lo, u);
    hi = max(hi, u);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    lo = min(lo, (uint32_t)__shfl_xor((int)lo, o));
    hi = max(hi, (uint32_t)__shfl_xor((int)hi, o));
  }
  if (lane == 0) {
    wmin[wave] = lo;
    wmax[wave] = hi;
  }
  __syncthreads();
  uint32_t kmin = wmin[0], kmax = wmax[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    kmin = min(kmin, wmin[w]);
    kmax = max(kmax, wmax[w]);
  }
  const int lz = kmax > kmin ? __clz(kmax - kmin) : 0;
  auto vkey = [&](uint32_t u) { return (u - kmin) << lz; };  // order-preserving on [kmin, kmax]
  uint32_t prefix = 0, pmask = 0;
  uint32_t kk = (uint32_t)k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int e = tid; e < kWaves * 256; e += kTopkThreads) (&hist[0][0])[e] = 0;
    __syncthreads();
    if (cached) {
#pragma unroll
      for (int j = 0; j < kTopkCache; ++j) {
        const uint32_t v = vkey(key[j]);
        if (i0 + j < i1 && (v & pmask) == prefix) atomicAdd(&hist[wave][(v >> shift) & 255u], 1u);
      }
    } else {
      for (int i = i0; i < i1; ++i) {
        const uint32_t v = vkey(order_key(s[i]));
        if ((v & pmask) == prefix) atomicAdd(&hist[wave][(v >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (tid < 256) {  // the waves' histograms summed per bucket
      uint32_t c = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) c += hist[w][tid];
      total[tid] = c;
    }
    __syncthreads();
    if (wave == 0) {
      // lane l owns buckets 255 - 4l .. 252 - 4l (descending); suffix counts by a wave scan
      uint32_t c[4], tot = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = total[255 - 4 * lane - j];
        tot += c[j];
      }
      uint32_t incl = tot;  // inclusive scan over lanes (higher buckets first)
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      const uint32_t before = incl - tot;
      // the lane whose buckets take the count past kk holds the k-th key
      if (before < kk && incl >= kk) {
        uint32_t cum = before;
        int bsel = 255 - 4 * lane - 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (cum + c[j] >= kk) {
            bsel = 255 - 4 * lane - j;
            break;
          }
          cum += c[j];
        }
        sh_k = kk - cum;
        sh_prefix = prefix | ((uint32_t)bsel << shift);
      }
    }
    __syncthreads();
    kk = sh_k;
    prefix = sh_prefix;
    pmask |= 255u << shift;
  }
  const uint32_t T = (prefix >> lz) + kmin;  // key of the k-th largest value
  int cg = 0, ce = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t u = key_at(i - i0);
    cg += u > T;
    ce += u == T;
  }
  // exclusive prefix counts over the threads (index order): a scan within each wave, then the
  // waves' totals
  int ig = cg, ie = ce;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int tg = __shfl_up(ig, o), te = __shfl_up(ie, o);
    if (lane >= o) {
      ig += tg;
      ie += te;
    }
  }
  if (lane == 63) {
    wsum_g[wave] = ig;
    wsum_e[wave] = ie;
  }
  __syncthreads();
  int base_g = 0, base_e = 0, total_g = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int g = wsum_g[w], e = wsum_e[w];
    base_g += w < wave ? g : 0;
    base_e += w < wave ? e : 0;
    total_g += g;
  }
  const int need_e = k - total_g;  // equal-key elements to take, lowest index first
  int eq_before = base_e + ie - ce;
  // selected before this thread's range = greater elements + min(equal, need)
  int pos = base_g + ig - cg + min(eq_before, need_e);
  for (int i = i0; i < i1; ++i) {
    const uint32_t u = key_at(i - i0);
    if (u > T) {
      out[pos++] = i;
    } else if (u == T) {
      if (eq_before < need_e) out[pos++] = i;
      ++eq_before;
    }
  }
}

}  // namespace

extern "C" size_t dkv_score_workspace_bytes(const dkv_attend_args_t* a) {
  if (check_attend(a, "dkv_score_workspace_bytes")) return 0;
  return make_score_layout(a).total;
}

extern "C" int dkv_score_begin(float* importance, int32_t n, void* stream) {
  DKV_REQUIRE(importance && n >= 0, DKV_EINVAL, "dkv_score_begin: bad arguments");
  if (n == 0) return DKV_OK;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((n + 255) / 256), dim3(256), 0, dkv::as_stream(stream), importance, n);
  return dkv::check_launch("dkv_score_begin");
}

extern "C" int dkv_score_layer(const dkv_attend_args_t* a, const float* key_question, float* importance,
                               void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_attend(a, "dkv_score_layer");
  if (rc) return rc;
  DKV_REQUIRE(a->batch == 1, DKV_ESHAPE, "dkv_score_layer: batch must be 1");
  DKV_REQUIRE(key_question && importance, DKV_EINVAL, "dkv_score_layer: null key_question / importance");
  int E = 0;
  if (a->cu_exact) {
    DKV_REQUIRE(a->cu_exact_host && a->key_exact, DKV_EINVAL, "dkv_score_layer: exact keys need host offsets");
    DKV_REQUIRE(a->exact_dtype == DKV_F32, DKV_EINVAL, "dkv_score_layer: exact keys must be f32 (exact_dtype %d)",
                a->exact_dtype);
    DKV_REQUIRE(a->cu_exact_host[0] == 0, DKV_ESHAPE, "dkv_score_layer: cu_exact[0] must be 0");
    E = a->cu_exact_host[1] - a->cu_exact_host[0];
  }
  const ScoreLayout S = make_score_layout(a);
  DKV_REQUIRE(workspace && workspace_bytes >= S.total, DKV_EWORKSPACE,
              "dkv_score_layer: workspace %zu B < required %zu B", workspace_bytes, S.total);
  char* ws = (char*)workspace;
  hipStream_t st = dkv::as_stream(stream);
  // layer parity picks the halves of the double buffers: this layer's K2 output and statistics go
  // to `cur`, the previous layer's wait in `prv` for their importance
  const int cur = a->layer & 1, prv = cur ^ 1;
  uint16_t* probs[2] = {(uint16_t*)(ws + S.base.probs), (uint16_t*)(ws + S.probs2)};
  rc = launch_keys_scores(a, S.base, ws, st, /*scoring=*/true, (float*)(ws + S.sub_max[cur]),
                          (float*)(ws + S.sub_sum), probs[cur]);
  if (rc) return rc;
  RowStatsArgs e{};
  e.query = a->query;
  e.key_exact = (const float*)a->key_exact;
  e.key_question = key_question;
  e.sub_max = (const float*)(ws + S.sub_max[cur]);
  e.sub_sum = (const float*)(ws + S.sub_sum);
  e.stat = (float*)(ws + S.stat[cur]);
  e.scaling = a->scaling;
  e.Hkv = a->kv_heads;
  e.Hq = a->q_heads;
  e.q_len = a->q_len;
  e.E = E;
  e.query_dtype = a->query_dtype;
  e.nsub = S.base.ntiles * 4;
  auto importance_args = [&](int buf) {
    ImportanceArgs im{};
    im.probs = probs[buf];
    im.sub_max = (const float*)(ws + S.sub_max[buf]);
    im.stat = (const float*)(ws + S.stat[buf]);
    im.importance = importance;
    im.R_total = S.base.R_total;
    im.n = S.base.n_total;
    im.ntiles = S.base.ntiles;
    return im;
  };
  // eight rows of one query head per statistics workgroup when the question length allows it
  const bool rows8 = a->q_len % 8 == 0;
  const int n_stat = rows8 ? S.base.R_total / 8 : S.base.R_total;
  const int n_imp = S.base.n_total > 0 ? S.base.ntiles * 4 : 0;
  auto launch = [&](int n_stat_wg, const ImportanceArgs& im, int n_imp_wg) {
    const dim3 grid((unsigned)(n_stat_wg + n_imp_wg)), block(kImpThreads);
    if (a->head_dim == 128) {
      if (rows8)
        hipLaunchKernelGGL((score_stats_kernel<128, 8>), grid, block, 0, st, e, im, n_stat_wg);
      else
        hipLaunchKernelGGL((score_stats_kernel<128, 1>), grid, block, 0, st, e, im, n_stat_wg);
    } else {
      if (rows8)
        hipLaunchKernelGGL((score_stats_kernel<64, 8>), grid, block, 0, st, e, im, n_stat_wg);
      else
        hipLaunchKernelGGL((score_stats_kernel<64, 1>), grid, block, 0, st, e, im, n_stat_wg);
    }
    return dkv::check_launch("score_stats");
  };
  // this layer's statistics, and the previous layer's importance (none before layer 0)
  rc = launch(n_stat, importance_args(prv), a->layer > 0 ? n_imp : 0);
  if (rc) return rc;
  // the last layer adds its own importance at once
  if (a->layer == a->layers - 1 && n_imp > 0) return launch(0, importance_args(cur), n_imp);
  return DKV_OK;
}

extern "C" size_t dkv_topk_workspace_bytes(int32_t n) {
  (void)n;
  return 0;
}

extern "C" int dkv_topk(const float* scores, int32_t n, int32_t k, int32_t* idx_out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  DKV_REQUIRE(scores && idx_out, DKV_EINVAL, "dkv_topk: null pointer");
  DKV_REQUIRE(n >= 0 && k >= 0 && k <= n, DKV_ESHAPE, "dkv_topk: need 0 <= k <= n (k=%d n=%d)", k, n);
  if (k == 0) return DKV_OK;
  hipLaunchKernelGGL(topk_kernel, dim3(1), dim3(kTopkThreads), 0, dkv::as_stream(stream), scores, n, k, idx_out);
  return dkv::check_launch("dkv_topk");
}

// ===========================================================================
// Allocation-free variant of dkv_attend_prepare + dkv_attend_layer, for
// callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid it).  The workspace is the
// file-scope device array below, `kStaticScratchBytes` per GPU, held by every
// GPU the library runs on until the process ends.  Every call on one GPU
// shares that GPU's array: each call decodes the codes again and rewrites
// every area it then reads (no area needs to start at zero: the decode writes
// every slot, K2 every tile statistic and probability the later kernels
// read, and K3a/K3b every partial), so calls in sequence are independent,
// but calls that overlap on one GPU (different streams or threads) race.
// ===========================================================================
namespace {

constexpr size_t kStaticScratchBytes = DKV_NOALLOC_MAX_BYTES;  // 64 MiB
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each GPU (null until looked up)

// The current device's address of `scratch`, looked up once per device with that device
// current (in host code the array's name is not a device address).
int scratch_address(void** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  DKV_REQUIRE(e == hipSuccess, DKV_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  DKV_REQUIRE(dev >= 0 && dev < kMaxDevices, DKV_EINVAL, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    DKV_REQUIRE(e == hipSuccess && p, DKV_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", what,
                hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DKV_OK;
}

}  // namespace

extern "C" int dkv_attend_layer_noalloc(const dkv_attend_args_t* a, void* stream) {
  int rc = check_attend(a, "dkv_attend_layer_noalloc");
  if (rc) return rc;
  int E_total = 0;
  rc = check_values(a, E_total);
  if (rc) return rc;
  const Layout L = make_layout(a);
  DKV_REQUIRE(L.total <= kStaticScratchBytes, DKV_EWORKSPACE,
              "dkv_attend_layer_noalloc: this context needs %zu B of scratch; the static maximum is %zu B "
              "(use dkv_attend_prepare + dkv_attend_layer with a caller workspace)",
              L.total, kStaticScratchBytes);
  void* ws = nullptr;
  rc = scratch_address(&ws, "dkv_attend_layer_noalloc");
  if (rc) return rc;
  rc = dkv_attend_prepare(a, 8, ws, kStaticScratchBytes, stream);
  if (rc) return rc;
  return dkv_attend_layer(a, ws, kStaticScratchBytes, stream);
}
