// One layer of attention directly over the packed bit-plane codes.
//
// Replaces scripts/compressed_attention.py:105-137 (CompressedContext._keys /
// attend) of SrikanthBalaaji/Dimmer-KV, applied to progressive codes
// (scripts/progressive.py:47-55, 196-201):
//
//   K2  keys_scores  : per (256-token tile, head group) - unpack the key codes
//                      of one 64-component group at a time into LDS as fp16,
//                      multiply by the layer's key-basis slice on MFMA
//                      (32x32x16 f16, fp32 accumulate), add the mean, apply
//                      RoPE at the token positions, score against the GQA
//                      query rows on MFMA, write fp32 scores and per-tile
//                      (max, sum exp) statistics.  Keys never reach HBM.
//   K3a value_weights: p~ = exp(s - M_c); per (token split, 4 groups) the
//                      value codes are unpacked and p~ @ C_v accumulated on
//                      MFMA -> partial coefficient-space outputs.
//   K3b basis_apply  : sum the partials, multiply once by the value basis of
//                      the KV head (per 128-component chunk).
//   K3c finish       : merge with the exact tokens (sinks, recent, new) in the
//                      same softmax, add sum(p) * mean_v, normalise, write.
#include <math.h>

#include "dkv_device.h"
#include "dkv_host.h"

namespace {

constexpr int kTileTok = 256;    // tokens per K2 workgroup
constexpr int kK2Threads = 512;  // 8 waves: 4 token quarters x 2 row halves
constexpr int kStride = 72;      // LDS row stride in halves for [row][64] tiles (64 + 8 pad)
constexpr int kSplitTok = 1024;  // tokens per K3a split
constexpr int kK3Threads = 256;  // 4 waves, one 64-component group each
constexpr int kVtStride = 40;    // LDS stride (halves) of the transposed value tile [64][32 + 8]
constexpr int kPStride = 40;     // LDS stride (halves) of the p~ tile [32][32 + 8]
constexpr int kChunk = 128;      // components per K3b workgroup

struct K2Args {
  dkv_stream_t key;
  const int32_t* cu_seqlens;
  const int32_t* positions;
  const uint16_t* key_basis;
  const float* mean_k;
  const float* rope_cos;
  const float* rope_sin;
  const void* query;
  float* scores;
  float* tile_max;
  float* tile_sum;
  float scaling;
  int batch, layer, Hkv, Hq, q_len, G, n_total, ntiles, total_wg, per_xcd, query_dtype;
};

DKV_DEVICE half8 lds_half8(const half_t* p) { return *(const half8*)p; }

DKV_DEVICE half8 load_query8(const void* q, long idx, int dtype) {
  half8 r;
  if (dtype == DKV_F16) {
    r = *(const half8*)((const half_t*)q + idx);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (half_t)load_as_float(q, idx + i, dtype);
  }
  return r;
}

// ---------------------------------------------------------------------------
// K2.  D = head_dim (64 or 128).  The workgroup covers HPW = 256 / D heads
// (256 basis rows); wave w takes tokens (w & 3) * 64 .. +64 and basis rows
// (w >> 2) * 128 .. +128 of the tile.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kK2Threads) void keys_scores_kernel(K2Args a) {
  constexpr int HPW = 256 / D;      // heads per workgroup
  constexpr int DB = D / 32;        // 32-row blocks per head
  constexpr int HALF_BLK = DB / 2;  // RoPE partner offset in blocks
  constexpr int KSTR = D + 8;       // LDS stride of the rebuilt-key tile
  __shared__ __attribute__((aligned(16))) half_t lds[2 * 2 * kTileTok * kStride];
  __shared__ float stat_m[HPW][4][32];
  __shared__ float stat_s[HPW][4][32];

  const int bid = blockIdx.x;
  const int lin = (bid & 7) * a.per_xcd + (bid >> 3);
  if (lin >= a.total_wg) return;
  const int nhg = a.Hkv / HPW;
  const int tile = lin / nhg, hg = lin % nhg;
  const int2 bt = find_tile(a.cu_seqlens, a.batch, kTileTok, tile);
  const int b = bt.x;
  const int tok0 = a.cu_seqlens[b] + bt.y * kTileTok;
  const int count = min(kTileTok, a.cu_seqlens[b + 1] - tok0);
  const int h0 = hg * HPW;
  const int G = a.G;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tq = wave & 3, hs = wave >> 2;
  const int l32 = lane & 31, lhi = lane >> 5;

  // Unpack role: token ut, half uh.
  const int ut = tid >> 1, uh = tid & 1;
  const bool uvalid = ut < count;
  const int ut_g = tok0 + ut;
  const int ukp = uvalid ? a.key.pieces[ut_g] : 0;
  const uint8_t* ubase = uvalid ? a.key.blob + a.key.tok_off[ut_g] : nullptr;
  const uint8_t* planes_row = a.key.order.planes + (long)ukp * G;
  const int32_t* seg_row = a.key.order.seg_off + (long)ukp * G;

  const uint16_t* basis_layer = a.key_basis + (long)a.layer * G * a.Hkv * D * 64 + (long)h0 * D * 64;
  const long basis_group_stride = (long)a.Hkv * D * 64;

  half_t* A0 = lds;                          // codes   [2][256][72]
  half_t* B0 = lds + 2 * kTileTok * kStride;  // basis   [2][256][72]

  floatx16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  uint32_t pl[8], header = 0u;
  int um = 0;
  uint4 br0, br1, br2, br3;

#define DKV_K2_ISSUE(g_)                                                              \
  do {                                                                                \
    um = uvalid ? (int)planes_row[(g_)] : 0;                                          \
    if (uvalid) {                                                                     \
      load_segment(ubase + seg_row[(g_)], um, uh, pl, header);                        \
    } else {                                                                          \
      _Pragma("unroll") for (int p_ = 0; p_ < 8; ++p_) pl[p_] = 0u;                   \
      header = 0u;                                                                    \
    }                                                                                 \
    const uint4* src_ = (const uint4*)(basis_layer + (long)(g_) * basis_group_stride); \
    br0 = src_[0 * kK2Threads + tid];                                                 \
    br1 = src_[1 * kK2Threads + tid];                                                 \
    br2 = src_[2 * kK2Threads + tid];                                                 \
    br3 = src_[3 * kK2Threads + tid];                                                 \
  } while (0)

#define DKV_K2_FINISH(buf_)                                                            \
  do {                                                                                 \
    const AffineDq dq_ = affine_from_header(header, um);                               \
    uint32_t vals_[16];                                                                \
    unpack_half_f16(pl, dq_, vals_);                                                   \
    uint4* dstA_ = (uint4*)(A0 + ((buf_) * kTileTok + ut) * kStride + uh * 32);        \
    dstA_[0] = make_uint4(vals_[0], vals_[1], vals_[2], vals_[3]);                     \
    dstA_[1] = make_uint4(vals_[4], vals_[5], vals_[6], vals_[7]);                     \
    dstA_[2] = make_uint4(vals_[8], vals_[9], vals_[10], vals_[11]);                   \
    dstA_[3] = make_uint4(vals_[12], vals_[13], vals_[14], vals_[15]);                 \
    half_t* bdst_ = B0 + (buf_) * kTileTok * kStride;                                  \
    *(uint4*)(bdst_ + ((0 * kK2Threads + tid) >> 3) * kStride + (tid & 7) * 8) = br0;  \
    *(uint4*)(bdst_ + ((1 * kK2Threads + tid) >> 3) * kStride + (tid & 7) * 8) = br1;  \
    *(uint4*)(bdst_ + ((2 * kK2Threads + tid) >> 3) * kStride + (tid & 7) * 8) = br2;  \
    *(uint4*)(bdst_ + ((3 * kK2Threads + tid) >> 3) * kStride + (tid & 7) * 8) = br3;  \
  } while (0)

  DKV_K2_ISSUE(0);
  DKV_K2_FINISH(0);
  for (int g = 0; g < G; ++g) {
    const int buf = g & 1;
    __syncthreads();
    if (g + 1 < G) DKV_K2_ISSUE(g + 1);
    const half_t* At = A0 + buf * kTileTok * kStride;
    const half_t* Bt = B0 + buf * kTileTok * kStride;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kof = ks * 16 + lhi * 8;
      half8 bop[2], aop[4];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) bop[tb] = lds_half8(At + (tq * 64 + tb * 32 + l32) * kStride + kof);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) aop[rb] = lds_half8(Bt + (hs * 128 + rb * 32 + l32) * kStride + kof);
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
          acc[tb][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[rb], bop[tb], acc[tb][rb], 0, 0, 0);
    }
    if (g + 1 < G) DKV_K2_FINISH(buf ^ 1);
  }
#undef DKV_K2_ISSUE
#undef DKV_K2_FINISH
  __syncthreads();

  // ---- epilogue 1: + mean, RoPE, rebuilt keys -> LDS as fp16 [head][token][D+8]
  half_t* Kl = lds;
  const float* mean_layer = a.mean_k + (long)a.layer * a.Hkv * D;
  const int half_d = D / 2;
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const int n = tq * 64 + tb * 32 + l32;
    const bool valid = n < count;
    const int pos = valid ? a.positions[tok0 + n] : 0;
    const float* cosr = a.rope_cos + (long)pos * half_d;
    const float* sinr = a.rope_sin + (long)pos * half_d;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      if ((rb % DB) >= HALF_BLK) continue;
      const int rb2 = rb + HALF_BLK;
      const int hl = hs * (128 / D) + rb / DB;
      const float* mh = mean_layer + (long)(h0 + hl) * D;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const int d0 = (rb % DB) * 32 + 8 * v4 + 4 * lhi;
        const float4 mlo = *(const float4*)(mh + d0);
        const float4 mhi = *(const float4*)(mh + d0 + half_d);
        float4 c = make_float4(1.f, 1.f, 1.f, 1.f), s = make_float4(0.f, 0.f, 0.f, 0.f);
        if (valid) {
          c = *(const float4*)(cosr + d0);
          s = *(const float4*)(sinr + d0);
        }
        const float ml[4] = {mlo.x, mlo.y, mlo.z, mlo.w};
        const float mhv[4] = {mhi.x, mhi.y, mhi.z, mhi.w};
        const float cv[4] = {c.x, c.y, c.z, c.w};
        const float sv[4] = {s.x, s.y, s.z, s.w};
        half4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float klo = acc[tb][rb][v4 * 4 + e] + ml[e];
          const float khi = acc[tb][rb2][v4 * 4 + e] + mhv[e];
          lo[e] = (half_t)(klo * cv[e] - khi * sv[e]);
          hi[e] = (half_t)(khi * cv[e] + klo * sv[e]);
        }
        *(half4*)(Kl + (hl * kTileTok + n) * KSTR + d0) = lo;
        *(half4*)(Kl + (hl * kTileTok + n) * KSTR + d0 + half_d) = hi;
      }
    }
  }
  __syncthreads();

  // ---- epilogue 2: scores = q . k * scaling on MFMA, per 32-row block.
  const int gq = a.Hq / a.Hkv;
  const int RH = gq * a.q_len;
  const int mblocks = (RH + 31) / 32;
  constexpr int HPWAVE = HPW / 2;  // heads handled by each wave in this phase
  for (int mb = 0; mb < mblocks; ++mb) {
#pragma unroll
    for (int hh = 0; hh < HPWAVE; ++hh) {
      const int hl = hs * HPWAVE + hh;
      const int h = h0 + hl;
      floatx16 sacc[2];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[tb][v] = 0.0f;
      const int r = mb * 32 + l32;
      const bool rvalid = r < RH;
      const int qh = h * gq + (rvalid ? r / a.q_len : 0);
      const int qi = rvalid ? r % a.q_len : 0;
      const long qbase = (((long)b * a.Hq + qh) * a.q_len + qi) * D;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const int kof = ks * 16 + lhi * 8;
        half8 qa;
        if (rvalid) {
          qa = load_query8(a.query, qbase + kof, a.query_dtype);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) qa[i] = (half_t)0.0f;
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          const half8 kb = lds_half8(Kl + (hl * kTileTok + tq * 64 + tb * 32 + l32) * KSTR + kof);
          sacc[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa, kb, sacc[tb], 0, 0, 0);
        }
      }
      // sacc[tb][v]: token tq*64 + tb*32 + l32, row mb*32 + 8*(v/4) + 4*lhi + (v&3)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = mb * 32 + 8 * (v >> 2) + 4 * lhi + (v & 3);
        float x[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          const int n = tq * 64 + tb * 32 + l32;
          const bool ok = (row < RH) && (n < count);
          x[tb] = ok ? sacc[tb][v] * a.scaling : -INFINITY;
          if (ok) a.scores[(long)(h * RH + row) * a.n_total + tok0 + n] = x[tb];
        }
        float mx = fmaxf(x[0], x[1]);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        float sm = 0.0f;
        if (mx != -INFINITY) sm = __expf(x[0] - mx) + __expf(x[1] - mx);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) sm += __shfl_xor(sm, o, 64);
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
        const long o = (long)((h0 + hl) * RH + row) * a.ntiles + tile;
        a.tile_max[o] = M;
        a.tile_sum[o] = S;
      }
    }
    __syncthreads();
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

struct K3aArgs {
  dkv_stream_t value;
  const int32_t* cu_seqlens;
  const float* scores;
  const float* tile_max;
  float* w_part;
  int batch, R_total, n_total, ntiles, G, rank, nsplits, row_blocks, nchunks_g;
};

__global__ __launch_bounds__(kK3Threads) void value_weights_kernel(K3aArgs a) {
  __shared__ __attribute__((aligned(16))) half_t Pt[32 * kPStride];
  __shared__ __attribute__((aligned(16))) half_t Vt[4][64 * kVtStride];
  __shared__ float Mrow[32];

  const int bid = blockIdx.x;
  const int rbk = bid % a.row_blocks;
  const int gc = (bid / a.row_blocks) % a.nchunks_g;
  const int sp = bid / (a.row_blocks * a.nchunks_g);
  const int2 bs = find_tile(a.cu_seqlens, a.batch, kSplitTok, sp);
  const int b = bs.x;
  const int tok0 = a.cu_seqlens[b] + bs.y * kSplitTok;
  const int count = min(kSplitTok, a.cu_seqlens[b + 1] - tok0);
  const int tb0 = tiles_before(a.cu_seqlens, b, kTileTok);
  const int ntb = (a.cu_seqlens[b + 1] - a.cu_seqlens[b] + kTileTok - 1) / kTileTok;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int G = a.G;
  const int g = gc * 4 + wave;
  const bool gvalid = g < G;

  if (tid < 32) {
    const int row = rbk * 32 + tid;
    float M = -INFINITY;
    if (row < a.R_total)
      for (int t = 0; t < ntb; ++t) M = fmaxf(M, a.tile_max[(long)row * a.ntiles + tb0 + t]);
    Mrow[tid] = M;
  }
  __syncthreads();

  floatx16 acc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[nb][v] = 0.0f;

  const int ut = lane >> 1, uh = lane & 1;
  for (int c0 = 0; c0 < count; c0 += 32) {
    // p~ tile [32 rows][32 tokens]
#pragma unroll
    for (int e = tid; e < 32 * 32; e += kK3Threads) {
      const int rr = e >> 5, t = e & 31;
      const int row = rbk * 32 + rr;
      float p = 0.0f;
      if (row < a.R_total && c0 + t < count) {
        const float M = Mrow[rr];
        p = __expf(a.scores[(long)row * a.n_total + tok0 + c0 + t] - M);
      }
      Pt[rr * kPStride + t] = (half_t)p;
    }
    // value codes of token c0 + ut, this wave's group -> transposed [coef][token]
    {
      const int t = c0 + ut;
      uint32_t pl[8], header = 0u;
      int m = 0;
      if (gvalid && t < count) {
        const int tg = tok0 + t;
        const int kp = a.value.pieces[tg];
        m = a.value.order.planes[(long)kp * G + g];
        const uint8_t* seg = a.value.blob + a.value.tok_off[tg] + a.value.order.seg_off[(long)kp * G + g];
        load_segment(seg, m, uh, pl, header);
      } else {
#pragma unroll
        for (int p = 0; p < 8; ++p) pl[p] = 0u;
      }
      const AffineDq dq = affine_from_header(header, m);
      uint32_t vals[16];
      unpack_half_f16(pl, dq, vals);
      half_t* col = Vt[wave] + uh * 32 * kVtStride + ut;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t v2 = vals[j];
        uint16_t lo16 = (uint16_t)(v2 & 0xffffu), hi16 = (uint16_t)(v2 >> 16);
        half_t hlo, hhi;
        __builtin_memcpy(&hlo, &lo16, 2);
        __builtin_memcpy(&hhi, &hi16, 2);
        col[(2 * j) * kVtStride] = hlo;
        col[(2 * j + 1) * kVtStride] = hhi;
      }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kof = ks * 16 + lhi * 8;
      const half8 pa = lds_half8(Pt + l32 * kPStride + kof);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const half8 vb = lds_half8(Vt[wave] + (nb * 32 + l32) * kVtStride + kof);
        acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, vb, acc[nb], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  if (!gvalid) return;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int row = rbk * 32 + 8 * (v >> 2) + 4 * lhi + (v & 3);
      if (row < a.R_total) a.w_part[((long)sp * a.R_total + row) * a.rank + g * 64 + nb * 32 + l32] = acc[nb][v];
    }
}

// ---------------------------------------------------------------------------
// K3b: per (sequence, KV head, 128-component chunk): sum partials over the
// sequence's splits, multiply by the value basis chunk [128][D].
// ---------------------------------------------------------------------------
struct K3bArgs {
  const int32_t* cu_seqlens;
  const float* w_part;
  const uint16_t* value_basis;
  float* out_part;
  int batch, layer, Hkv, Hq, q_len, D, rank, R_total, nchunks;
};

__global__ __launch_bounds__(256) void basis_apply_kernel(K3bArgs a) {
  __shared__ float W[8][kChunk];
  __shared__ float red[256 / 64][8][128];
  const int c = blockIdx.x % a.nchunks;
  const int h = (blockIdx.x / a.nchunks) % a.Hkv;
  const int b = blockIdx.x / (a.nchunks * a.Hkv);
  const int tid = threadIdx.x;
  const int gq = a.Hq / a.Hkv;
  const int RH = gq * a.q_len;
  const int sp0 = tiles_before(a.cu_seqlens, b, kSplitTok);
  const int nsp = (a.cu_seqlens[b + 1] - a.cu_seqlens[b] + kSplitTok - 1) / kSplitTok;
  const int D = a.D;
  const int parts = 256 / D;  // threads per d
  const int d = tid % D, part = tid / D;
  const int ilen = kChunk / parts;
  const uint16_t* bv = a.value_basis + (((long)a.layer * a.Hkv + h) * a.rank + (long)c * kChunk) * D;
  for (int r0 = 0; r0 < RH; r0 += 8) {
    const int nr = min(8, RH - r0);
    for (int e = tid; e < nr * kChunk; e += 256) {
      const int rr = e / kChunk, i = e % kChunk;
      const long row = (long)h * RH + r0 + rr;
      float s = 0.0f;
      for (int sp = 0; sp < nsp; ++sp) s += a.w_part[((long)(sp0 + sp) * a.R_total + row) * a.rank + c * kChunk + i];
      W[rr][i] = s;
    }
    __syncthreads();
    float accr[8];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) accr[rr] = 0.0f;
    for (int i = part * ilen; i < (part + 1) * ilen; ++i) {
      const float bvv = half_bits_to_float(bv[(long)i * D + d]);
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) accr[rr] += W[rr][i] * bvv;
    }
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) red[part][rr][d] = accr[rr];
    __syncthreads();
    for (int e = tid; e < nr * D; e += 256) {
      const int rr = e / D, dd = e % D;
      float s = 0.0f;
      for (int p = 0; p < parts; ++p) s += red[p][rr][dd];
      a.out_part[(((long)c * a.batch + b) * a.R_total + (long)h * RH + r0 + rr) * D + dd] = s;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// K3c: one workgroup per (sequence, output row): exact tokens, softmax merge,
// mean term, normalisation.
// ---------------------------------------------------------------------------
struct K3cArgs {
  const int32_t* cu_seqlens;
  const int32_t* cu_exact;
  const float* tile_max;
  const float* tile_sum;
  const float* out_part;
  const float* mean_v;
  const float* key_exact;
  const float* value_exact;
  const float* mask;
  const void* query;
  void* out;
  float scaling;
  int batch, layer, Hkv, Hq, q_len, D, R_total, ntiles, nchunks, E_total, query_dtype, out_dtype;
};

constexpr int kMaxExact = 1024;

__global__ __launch_bounds__(128) void finish_kernel(K3cArgs a) {
  __shared__ float q[128];
  __shared__ float se[kMaxExact];
  __shared__ float red[128];
  __shared__ float bc[4];
  const int row = blockIdx.x % a.R_total;
  const int b = blockIdx.x / a.R_total;
  const int tid = threadIdx.x;
  const int D = a.D;
  const int gq = a.Hq / a.Hkv;
  const int qh = row / a.q_len, qi = row % a.q_len;
  const int h = qh / gq;
  const int tb0 = tiles_before(a.cu_seqlens, b, kTileTok);
  const int ntb = (a.cu_seqlens[b + 1] - a.cu_seqlens[b] + kTileTok - 1) / kTileTok;

  // compressed-part statistics
  float m = -INFINITY;
  for (int t = tid; t < ntb; t += 128) m = fmaxf(m, a.tile_max[(long)row * a.ntiles + tb0 + t]);
  red[tid] = m;
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  const float Mc = red[0];
  __syncthreads();
  float l = 0.0f;
  if (Mc != -INFINITY)
    for (int t = tid; t < ntb; t += 128) {
      const float mt = a.tile_max[(long)row * a.ntiles + tb0 + t];
      if (mt != -INFINITY) l += a.tile_sum[(long)row * a.ntiles + tb0 + t] * __expf(mt - Mc);
    }
  red[tid] = l;
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  const float Lc = red[0];
  __syncthreads();

  // exact tokens
  const int e0 = a.cu_exact ? a.cu_exact[b] : 0;
  const int E = a.cu_exact ? a.cu_exact[b + 1] - e0 : 0;
  if (tid < D) q[tid] = load_as_float(a.query, (((long)b * a.Hq + qh) * a.q_len + qi) * D + tid, a.query_dtype);
  __syncthreads();
  float me = -INFINITY;
  for (int j = tid; j < E; j += 128) {
    const float* kr = a.key_exact + ((long)h * a.E_total + e0 + j) * D;
    float dot = 0.0f;
    for (int dd = 0; dd < D; ++dd) dot += q[dd] * kr[dd];
    float s = dot * a.scaling;
    if (a.mask) s += a.mask[(long)qi * E + j];
    se[j] = s;
    me = fmaxf(me, s);
  }
  red[tid] = me;
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  const float Me = red[0];
  __syncthreads();
  const float M = fmaxf(Mc, Me);
  if (tid == 0) {
    bc[0] = (M == -INFINITY || Mc == -INFINITY) ? 0.0f : __expf(Mc - M);
    bc[1] = M;
  }
  __syncthreads();
  const float ec = bc[0];
  float le = 0.0f;
  for (int j = tid; j < E; j += 128) {
    const float w = (M == -INFINITY || se[j] == -INFINITY) ? 0.0f : __expf(se[j] - M);
    se[j] = w;
    le += w;
  }
  red[tid] = le;
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  const float Le = red[0];
  const float denom = ec * Lc + Le;
  if (tid < D) {
    float vc = 0.0f;
    for (int c = 0; c < a.nchunks; ++c) vc += a.out_part[(((long)c * a.batch + b) * a.R_total + row) * D + tid];
    vc += Lc * a.mean_v[((long)a.layer * a.Hkv + h) * D + tid];
    float ve = 0.0f;
    for (int j = 0; j < E; ++j) ve += se[j] * a.value_exact[((long)h * a.E_total + e0 + j) * D + tid];
    const float o = denom > 0.0f ? (ec * vc + ve) / denom : 0.0f;
    store_from_float(a.out, (((long)b * a.q_len + qi) * a.Hq + qh) * D + tid, a.out_dtype, o);
  }
}

// ---------------------------------------------------------------------------
// Workspace layout and argument checks.
// ---------------------------------------------------------------------------
struct Layout {
  int ntiles, nsplits, R_total, nchunks, n_total;
  size_t scores, tile_max, tile_sum, w_part, out_part, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Layout make_layout(const dkv_attend_args_t* a) {
  Layout L{};
  L.ntiles = 0;
  L.nsplits = 0;
  for (int b = 0; b < a->batch; ++b) {
    const int len = a->cu_seqlens_host[b + 1] - a->cu_seqlens_host[b];
    L.ntiles += (len + kTileTok - 1) / kTileTok;
    L.nsplits += (len + kSplitTok - 1) / kSplitTok;
  }
  L.n_total = a->cu_seqlens_host[a->batch];
  L.R_total = a->q_heads * a->q_len;
  L.nchunks = a->rank / kChunk;
  size_t off = 0;
  L.scores = off;
  off += align256((size_t)L.R_total * L.n_total * 4);
  L.tile_max = off;
  off += align256((size_t)L.R_total * L.ntiles * 4);
  L.tile_sum = off;
  off += align256((size_t)L.R_total * L.ntiles * 4);
  L.w_part = off;
  off += align256((size_t)L.nsplits * L.R_total * a->rank * 4);
  L.out_part = off;
  off += align256((size_t)L.nchunks * a->batch * L.R_total * a->head_dim * 4);
  L.total = off;
  return L;
}

int check_attend(const dkv_attend_args_t* a, const char* what) {
  DKV_REQUIRE(a, DKV_EINVAL, "%s: args is null", what);
  int rc = dkv::check_stream(&a->key, what);
  if (rc) return rc;
  DKV_REQUIRE(a->head_dim == 64 || a->head_dim == 128, DKV_ESHAPE, "%s: head_dim must be 64 or 128 (got %d)", what,
              a->head_dim);
  DKV_REQUIRE(a->rank > 0 && a->rank % kChunk == 0 && a->rank == 64 * a->key.order.groups, DKV_ESHAPE,
              "%s: rank %d must be a multiple of 128 and equal 64 * groups (%d)", what, a->rank,
              a->key.order.groups);
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
  DKV_REQUIRE(a->cu_seqlens_host[0] == 0, DKV_ESHAPE, "%s: cu_seqlens[0] must be 0", what);
  for (int b = 0; b < a->batch; ++b)
    DKV_REQUIRE(a->cu_seqlens_host[b + 1] >= a->cu_seqlens_host[b], DKV_ESHAPE, "%s: cu_seqlens not monotone", what);
  return DKV_OK;
}

int launch_keys_scores(const dkv_attend_args_t* a, const Layout& L, char* ws, hipStream_t st) {
  if (L.ntiles == 0) return DKV_OK;
  K2Args k{};
  k.key = a->key;
  k.cu_seqlens = a->cu_seqlens;
  k.positions = a->positions;
  k.key_basis = a->key_basis;
  k.mean_k = a->mean_k;
  k.rope_cos = a->rope_cos;
  k.rope_sin = a->rope_sin;
  k.query = a->query;
  k.scores = (float*)(ws + L.scores);
  k.tile_max = (float*)(ws + L.tile_max);
  k.tile_sum = (float*)(ws + L.tile_sum);
  k.scaling = a->scaling;
  k.batch = a->batch;
  k.layer = a->layer;
  k.Hkv = a->kv_heads;
  k.Hq = a->q_heads;
  k.q_len = a->q_len;
  k.G = a->key.order.groups;
  k.n_total = L.n_total;
  k.ntiles = L.ntiles;
  k.query_dtype = a->query_dtype;
  const int HPW = 256 / a->head_dim;
  k.total_wg = L.ntiles * (a->kv_heads / HPW);
  k.per_xcd = (k.total_wg + 7) / 8;
  const dim3 grid(8 * k.per_xcd);
  if (a->head_dim == 128)
    hipLaunchKernelGGL(keys_scores_kernel<128>, grid, dim3(kK2Threads), 0, st, k);
  else
    hipLaunchKernelGGL(keys_scores_kernel<64>, grid, dim3(kK2Threads), 0, st, k);
  return dkv::check_launch("keys_scores");
}

}  // namespace

extern "C" size_t dkv_attend_workspace_bytes(const dkv_attend_args_t* a) {
  if (check_attend(a, "dkv_attend_workspace_bytes")) return 0;
  return make_layout(a).total;
}

extern "C" int dkv_attend_layer(const dkv_attend_args_t* a, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_attend(a, "dkv_attend_layer");
  if (rc) return rc;
  rc = dkv::check_stream(&a->value, "dkv_attend_layer(value)");
  if (rc) return rc;
  DKV_REQUIRE(a->value.order.groups == a->key.order.groups, DKV_ESHAPE, "dkv_attend_layer: K/V group mismatch");
  DKV_REQUIRE(a->value_basis && a->mean_v && a->out, DKV_EINVAL, "dkv_attend_layer: null value/out pointer");
  DKV_REQUIRE(a->out_dtype >= DKV_F32 && a->out_dtype <= DKV_BF16, DKV_EINVAL, "dkv_attend_layer: bad out dtype");
  DKV_REQUIRE(!a->mask || a->batch == 1, DKV_ESHAPE, "dkv_attend_layer: mask is only supported for batch == 1");
  DKV_REQUIRE(!a->cu_exact || (a->key_exact && a->value_exact), DKV_EINVAL,
              "dkv_attend_layer: exact keys/values missing");
  const Layout L = make_layout(a);
  DKV_REQUIRE(workspace && workspace_bytes >= L.total, DKV_EWORKSPACE,
              "dkv_attend_layer: workspace %zu B < required %zu B", workspace_bytes, L.total);
  // The finish kernel keeps one sequence's exact scores in LDS.
  int E_total = 0;
  if (a->cu_exact) {
    DKV_REQUIRE(a->cu_exact_host, DKV_EINVAL, "dkv_attend_layer: cu_exact needs cu_exact_host");
    for (int b = 0; b < a->batch; ++b) {
      const int e = a->cu_exact_host[b + 1] - a->cu_exact_host[b];
      DKV_REQUIRE(e >= 0 && e <= kMaxExact, DKV_ESHAPE, "dkv_attend_layer: %d exact tokens (max %d)", e, kMaxExact);
    }
    E_total = a->cu_exact_host[a->batch];
  }
  char* ws = (char*)workspace;
  hipStream_t st = dkv::as_stream(stream);
  rc = launch_keys_scores(a, L, ws, st);
  if (rc) return rc;
  const int G = a->key.order.groups;
  if (L.nsplits > 0) {
    K3aArgs k{};
    k.value = a->value;
    k.cu_seqlens = a->cu_seqlens;
    k.scores = (const float*)(ws + L.scores);
    k.tile_max = (const float*)(ws + L.tile_max);
    k.w_part = (float*)(ws + L.w_part);
    k.batch = a->batch;
    k.R_total = L.R_total;
    k.n_total = L.n_total;
    k.ntiles = L.ntiles;
    k.G = G;
    k.rank = a->rank;
    k.nsplits = L.nsplits;
    k.row_blocks = (L.R_total + 31) / 32;
    k.nchunks_g = (G + 3) / 4;
    const long blocks = (long)L.nsplits * k.row_blocks * k.nchunks_g;
    hipLaunchKernelGGL(value_weights_kernel, dim3((unsigned)blocks), dim3(kK3Threads), 0, st, k);
    rc = dkv::check_launch("value_weights");
    if (rc) return rc;
  }
  K3bArgs kb{};
  kb.cu_seqlens = a->cu_seqlens;
  kb.w_part = (const float*)(ws + L.w_part);
  kb.value_basis = a->value_basis;
  kb.out_part = (float*)(ws + L.out_part);
  kb.batch = a->batch;
  kb.layer = a->layer;
  kb.Hkv = a->kv_heads;
  kb.Hq = a->q_heads;
  kb.q_len = a->q_len;
  kb.D = a->head_dim;
  kb.rank = a->rank;
  kb.R_total = L.R_total;
  kb.nchunks = L.nchunks;
  hipLaunchKernelGGL(basis_apply_kernel, dim3(a->batch * a->kv_heads * L.nchunks), dim3(256), 0, st, kb);
  rc = dkv::check_launch("basis_apply");
  if (rc) return rc;
  K3cArgs kc{};
  kc.cu_seqlens = a->cu_seqlens;
  kc.cu_exact = a->cu_exact;
  kc.tile_max = (const float*)(ws + L.tile_max);
  kc.tile_sum = (const float*)(ws + L.tile_sum);
  kc.out_part = (const float*)(ws + L.out_part);
  kc.mean_v = a->mean_v;
  kc.key_exact = a->key_exact;
  kc.value_exact = a->value_exact;
  kc.mask = a->mask;
  kc.query = a->query;
  kc.out = a->out;
  kc.scaling = a->scaling;
  kc.batch = a->batch;
  kc.layer = a->layer;
  kc.Hkv = a->kv_heads;
  kc.Hq = a->q_heads;
  kc.q_len = a->q_len;
  kc.D = a->head_dim;
  kc.R_total = L.R_total;
  kc.ntiles = L.ntiles;
  kc.nchunks = L.nchunks;
  kc.E_total = E_total;
  kc.query_dtype = a->query_dtype;
  kc.out_dtype = a->out_dtype;
  hipLaunchKernelGGL(finish_kernel, dim3(a->batch * L.R_total), dim3(128), 0, st, kc);
  return dkv::check_launch("finish");
}

// ===========================================================================
// K4a: question scoring of the hot tier (scripts/progressive.py:239-254 with
// scripts/dimmer.py:52-66).  Per layer: K2 scores every (query head, query
// position) row against the compressed keys; exact_stats adds the softmax
// mass of the exact context tokens and of the question's own keys (causal);
// importance_part accumulates sum over rows of p = exp(s - M) / L per token;
// importance_add folds the row-chunk partials into importance[n] in a fixed
// order, so results do not depend on scheduling.
// ===========================================================================
namespace {

constexpr int kRowChunk = 64;  // rows per importance_part workgroup
constexpr int kTokChunk = 256;

struct ExactStatsArgs {
  const void* query;
  const float* key_exact;     // [Hkv][E][D]
  const float* key_question;  // [Hkv][Lq][D]
  float* stat;                // [R_total][2] (max, sum exp)
  float scaling;
  int Hkv, Hq, q_len, D, E, query_dtype;
};

__global__ __launch_bounds__(128) void exact_stats_kernel(ExactStatsArgs a) {
  __shared__ float q[128];
  __shared__ float red[128];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int gq = a.Hq / a.Hkv;
  const int qh = row / a.q_len, qi = row % a.q_len;
  const int h = qh / gq;
  const int D = a.D;
  if (tid < D) q[tid] = load_as_float(a.query, ((long)qh * a.q_len + qi) * D + tid, a.query_dtype);
  __syncthreads();
  const int nkeys = a.E + qi + 1;  // exact context tokens + question keys 0..qi
  float m = -INFINITY;
  for (int j = tid; j < nkeys; j += 128) {
    const float* kr = j < a.E ? a.key_exact + ((long)h * a.E + j) * D
                              : a.key_question + ((long)h * a.q_len + (j - a.E)) * D;
    float dot = 0.0f;
    for (int d = 0; d < D; ++d) dot += q[d] * kr[d];
    m = fmaxf(m, dot * a.scaling);
  }
  red[tid] = m;
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  const float M = red[0];
  __syncthreads();
  float l = 0.0f;
  for (int j = tid; j < nkeys; j += 128) {
    const float* kr = j < a.E ? a.key_exact + ((long)h * a.E + j) * D
                              : a.key_question + ((long)h * a.q_len + (j - a.E)) * D;
    float dot = 0.0f;
    for (int d = 0; d < D; ++d) dot += q[d] * kr[d];
    l += __expf(dot * a.scaling - M);
  }
  red[tid] = l;
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  if (tid == 0) {
    a.stat[2 * row] = M;
    a.stat[2 * row + 1] = red[0];
  }
}

struct ImportanceArgs {
  const float* scores;  // [R_total][n]
  const float* tile_max;
  const float* tile_sum;
  const float* stat;  // [R_total][2]
  float* part;        // [nrc][n]
  int R_total, n, ntiles;
};

__global__ __launch_bounds__(kTokChunk) void importance_part_kernel(ImportanceArgs a) {
  __shared__ float Mr[kRowChunk];
  __shared__ float invL[kRowChunk];
  const int ntc = (a.n + kTokChunk - 1) / kTokChunk;
  const int tc = blockIdx.x % ntc, rc = blockIdx.x / ntc;
  const int tid = threadIdx.x;
  const int r0 = rc * kRowChunk;
  const int nr = min(kRowChunk, a.R_total - r0);
  if (tid < nr) {
    const int row = r0 + tid;
    float Mc = -INFINITY;
    for (int t = 0; t < a.ntiles; ++t) Mc = fmaxf(Mc, a.tile_max[(long)row * a.ntiles + t]);
    float Lc = 0.0f;
    if (Mc != -INFINITY)
      for (int t = 0; t < a.ntiles; ++t) {
        const float mt = a.tile_max[(long)row * a.ntiles + t];
        if (mt != -INFINITY) Lc += a.tile_sum[(long)row * a.ntiles + t] * __expf(mt - Mc);
      }
    const float Me = a.stat[2 * row], Le = a.stat[2 * row + 1];
    const float M = fmaxf(Mc, Me);
    float L = 0.0f;
    if (Mc != -INFINITY) L += Lc * __expf(Mc - M);
    if (Me != -INFINITY) L += Le * __expf(Me - M);
    Mr[tid] = M;
    invL[tid] = L > 0.0f ? 1.0f / L : 0.0f;
  }
  __syncthreads();
  const int tok = tc * kTokChunk + tid;
  if (tok >= a.n) return;
  float acc = 0.0f;
  for (int r = 0; r < nr; ++r) acc += __expf(a.scores[(long)(r0 + r) * a.n + tok] - Mr[r]) * invL[r];
  a.part[(long)rc * a.n + tok] = acc;
}

__global__ __launch_bounds__(256) void importance_add_kernel(const float* __restrict__ part, int nrc, int n,
                                                             float* __restrict__ importance) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float s = 0.0f;
  for (int r = 0; r < nrc; ++r) s += part[(long)r * n + i];
  importance[i] += s;
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

struct ScoreLayout {
  Layout base;
  size_t stat, part, total;
  int nrc;
};

ScoreLayout make_score_layout(const dkv_attend_args_t* a) {
  ScoreLayout S{};
  S.base = make_layout(a);
  size_t off = S.base.w_part;  // scores + tile stats are shared with the attend layout
  S.stat = off;
  off += align256((size_t)S.base.R_total * 2 * 4);
  S.nrc = (S.base.R_total + kRowChunk - 1) / kRowChunk;
  S.part = off;
  off += align256((size_t)S.nrc * S.base.n_total * 4);
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

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ s, int n, int k,
                                                            int32_t* __restrict__ out) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sh_prefix, sh_k;
  __shared__ int scan_g[kTopkThreads];
  __shared__ int scan_e[kTopkThreads];
  const int tid = threadIdx.x;
  const int per = (n + kTopkThreads - 1) / kTopkThreads;
  const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
  uint32_t prefix = 0, pmask = 0;
  uint32_t kk = (uint32_t)k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int i = i0; i < i1; ++i) {
      const uint32_t u = order_key(s[i]);
      if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t cum = 0;
      int bsel = 0;
      for (int bb = 255; bb >= 0; --bb) {
        if (cum + hist[bb] >= kk) {
          bsel = bb;
          break;
        }
        cum += hist[bb];
      }
      sh_k = kk - cum;
      sh_prefix = prefix | ((uint32_t)bsel << shift);
    }
    __syncthreads();
    kk = sh_k;
    prefix = sh_prefix;
    pmask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t T = prefix;  // key of the k-th largest value
  int cg = 0, ce = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t u = order_key(s[i]);
    cg += u > T;
    ce += u == T;
  }
  scan_g[tid] = cg;
  scan_e[tid] = ce;
  __syncthreads();
  // inclusive scans (Hillis-Steele)
  for (int o = 1; o < kTopkThreads; o <<= 1) {
    const int vg = tid >= o ? scan_g[tid - o] : 0;
    const int ve = tid >= o ? scan_e[tid - o] : 0;
    __syncthreads();
    scan_g[tid] += vg;
    scan_e[tid] += ve;
    __syncthreads();
  }
  const int total_g = scan_g[kTopkThreads - 1];
  const int need_e = k - total_g;  // equal-key elements to take, lowest index first
  int eq_before = scan_e[tid] - ce;
  int g_before = scan_g[tid] - cg;
  // selected before this thread's range = greater elements + min(equal, need)
  int pos = g_before + min(eq_before, need_e);
  for (int i = i0; i < i1; ++i) {
    const uint32_t u = order_key(s[i]);
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
    E = a->cu_exact_host[1] - a->cu_exact_host[0];
  }
  const ScoreLayout S = make_score_layout(a);
  DKV_REQUIRE(workspace && workspace_bytes >= S.total, DKV_EWORKSPACE,
              "dkv_score_layer: workspace %zu B < required %zu B", workspace_bytes, S.total);
  char* ws = (char*)workspace;
  hipStream_t st = dkv::as_stream(stream);
  rc = launch_keys_scores(a, S.base, ws, st);
  if (rc) return rc;
  ExactStatsArgs e{};
  e.query = a->query;
  e.key_exact = a->key_exact;
  e.key_question = key_question;
  e.stat = (float*)(ws + S.stat);
  e.scaling = a->scaling;
  e.Hkv = a->kv_heads;
  e.Hq = a->q_heads;
  e.q_len = a->q_len;
  e.D = a->head_dim;
  e.E = E;
  e.query_dtype = a->query_dtype;
  hipLaunchKernelGGL(exact_stats_kernel, dim3(S.base.R_total), dim3(128), 0, st, e);
  rc = dkv::check_launch("exact_stats");
  if (rc) return rc;
  const int n = S.base.n_total;
  if (n == 0) return DKV_OK;
  ImportanceArgs im{};
  im.scores = (const float*)(ws + S.base.scores);
  im.tile_max = (const float*)(ws + S.base.tile_max);
  im.tile_sum = (const float*)(ws + S.base.tile_sum);
  im.stat = (const float*)(ws + S.stat);
  im.part = (float*)(ws + S.part);
  im.R_total = S.base.R_total;
  im.n = n;
  im.ntiles = S.base.ntiles;
  const int ntc = (n + kTokChunk - 1) / kTokChunk;
  hipLaunchKernelGGL(importance_part_kernel, dim3(ntc * S.nrc), dim3(kTokChunk), 0, st, im);
  rc = dkv::check_launch("importance_part");
  if (rc) return rc;
  hipLaunchKernelGGL(importance_add_kernel, dim3((n + 255) / 256), dim3(256), 0, st, (const float*)(ws + S.part),
                     S.nrc, n, importance);
  return dkv::check_launch("importance_add");
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
