/*
 * dimmerkv.h - C ABI of libdimmerkv_hip.so, the MI355X (gfx950) kernels for
 * Dimmer-KV's answer-time path: decode attention run directly over a
 * per-token variable-precision, bit-plane-coded, cross-layer-PCA KV cache.
 *
 * The reference (SrikanthBalaaji/Dimmer-KV) is pure Python on PyTorch; its
 * "interface" for this path is a set of Python functions.  Each entry point
 * below names the reference function whose work it replaces.  The Python
 * modules in dimmer-kv_amd/ (progressive.py, compressed_attention.py,
 * methods.py, dimmer.py) keep the reference's API and call these through
 * ctypes.
 *
 * Conventions
 * - Every pointer in a struct or argument is a device pointer unless its
 *   comment says "host".
 * - The library never allocates or frees memory.  Kernels that need scratch
 *   memory take a caller-provided workspace sized by the matching
 *   *_workspace_bytes() query.  Calls that overlap on different streams
 *   need separate workspaces.
 * - Calls are asynchronous on the given stream (hipStream_t passed as void*;
 *   NULL = the default stream) and never synchronise the host.
 * - Every entry point validates its arguments before launching anything and
 *   returns 0 on success or a negative DKV_E* code; dkv_last_error() then
 *   holds a message (thread-local).
 */
#ifndef DIMMERKV_H
#define DIMMERKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DKV_ABI_VERSION 3  /* 3: dkv_attend_args_t.exact_dtype; 2: dkv_stream_t.format */

/* Status codes.  The Python wrapper maps them to the reference's exception
 * types: DKV_EINVAL/DKV_ESHAPE -> ValueError, DKV_EBUDGET -> AssertionError,
 * DKV_ELAUNCH/DKV_EWORKSPACE -> RuntimeError. */
#define DKV_OK 0
#define DKV_EINVAL (-1)     /* null pointer or bad enum */
#define DKV_ESHAPE (-2)     /* inconsistent sizes */
#define DKV_EWORKSPACE (-3) /* workspace too small */
#define DKV_ELAUNCH (-4)    /* hipGetLastError after launch */
#define DKV_EBUDGET (-5)    /* byte budget exceeded */

/* Element types of query / output / dequantized coefficients. */
#define DKV_F32 0
#define DKV_F16 1
#define DKV_BF16 2

/* Progressive order of one stream (scripts/progressive.py:58-64 Order):
 * the per-token plane map is planes[pieces[t]].  seg_off / cold_off are
 * derived tables (byte offset of group g's segment in a hot / cold token blob
 * whose hot prefix is k pieces); prefix_bytes[k] is the hot blob size. */
typedef struct dkv_order {
  int32_t groups;              /* G = rank / 64 */
  int32_t pieces;              /* K = number of (group, plane) pieces, <= 8G */
  const uint8_t* planes;       /* [K+1][G] */
  const int32_t* seg_off;      /* [K+1][G] */
  const int32_t* cold_off;     /* [K+1][G] */
  const int32_t* prefix_bytes; /* [K+1] */
} dkv_order_t;

/* kvtc rung ladder of one stream (scripts/kvtc.py:100-105 Stream.rungs /
 * rung_bytes): bits[r][g] in {0, 2, 4, 8} is the width of group g at rung r.
 * seg_off[r][g] is the byte offset of group g's segment in a token blob at
 * rung r and rung_bytes[r] the blob size (scripts/kvtc.py:82-85: 8b bytes of
 * codes + 4 B of shift/scale per group with b > 0). */
typedef struct dkv_ladder {
  int32_t groups;              /* G = rank / 64 */
  int32_t rungs;               /* R (rows of the tables) */
  const uint8_t* bits;         /* [R][G] */
  const int32_t* seg_off;      /* [R][G] */
  const int32_t* rung_bytes;   /* [R] */
} dkv_ladder_t;

/* Stream formats. */
#define DKV_FMT_PLANES 0 /* progressive bit planes (scripts/progressive.py) */
#define DKV_FMT_LADDER 1 /* kvtc ladder codes (scripts/kvtc.py, scripts/kvtc_storage.py) */

/* One stream (keys or values) of a packed hot tier; token t's blob starts at
 * blob + tok_off[t].
 *
 * DKV_FMT_PLANES: the blob holds pieces[t] pieces (prefix_bytes[pieces[t]]
 * bytes).  Layout: for every group with m > 0 planes, [low f16][span f16][m
 * plane words of 8 B].  A plane word is two little-endian u32 halves;
 * coefficient 32h + 4w + i (w < 8, i < 4) of plane p (0 = most significant
 * bit) sits at bit (8i + w + 7 - p) mod 32 of half h.
 *
 * DKV_FMT_LADDER: pieces[t] is the token's rung r (ladder.bits row) and the
 * blob holds rung_bytes[r] bytes: for every group with b > 0 bits,
 * [low f16][scale f16][64 codes of b bits, LSB-first: code j at bit b*j of the
 * segment's code bytes] (the packing of scripts/kvtc_storage.py:21-27 applied
 * per (token, group)); the coefficient is code * scale + low in fp32
 * (scripts/kvtc.py:74-78), 0 for a group with b = 0.  `order` is unused. */
typedef struct dkv_stream {
  const uint8_t* blob;
  const int64_t* tok_off; /* [n] */
  const int16_t* pieces;  /* [n] */
  dkv_order_t order;
  int32_t format;         /* DKV_FMT_* */
  dkv_ladder_t ladder;
} dkv_stream_t;

int dkv_abi_version(void);
const char* dkv_last_error(void);

/* ---- packing (encoder side; scripts/progressive.py:103-110 TokenStore,
 *      byte accounting :185-194) ------------------------------------------ */

/* codes u8 [n][G][64], low/span f16 [n][G], pieces [n] -> hot blob at
 * hot_off[t] and cold blob at cold_off[t] (both int64 [n], byte offsets).
 * The cold blob of a token is [low,span if m==0][planes m..7] per group. */
int dkv_pack_planes(const uint8_t* codes, const uint16_t* low, const uint16_t* span, const int16_t* pieces,
                    int32_t n, dkv_order_t order, uint8_t* hot, const int64_t* hot_off, uint8_t* cold,
                    const int64_t* cold_off, void* stream);

/* codes u8 [n][G][64] (below 2^bits), low/scale f16 [n][G], rung [n] ->
 * ladder blobs at tok_off[t] (int64 [n]) in the DKV_FMT_LADDER layout
 * (replaces the per-rung code sections of scripts/kvtc_storage.py:63-75 with
 * one self-contained blob per token, so any token decodes on its own). */
int dkv_pack_ladder(const uint8_t* codes, const uint16_t* low, const uint16_t* scale, const int16_t* rung,
                    int32_t n, dkv_ladder_t ladder, uint8_t* blob, const int64_t* tok_off, void* stream);

/* ---- byte storage (replaces the per-rung code sections of
 *      scripts/kvtc_storage.py:56-75 encode_bytes and :98-119 decode_bytes) ---
 * The storage layout of one stream's compressed tokens: for every rung (in
 * increasing order) and every width w in 2, 4, 8 that the rung uses, one
 * section holding, for the tokens of the rung in increasing order and the
 * groups of width w in increasing order, first all the codes (64 per group,
 * w bits each, LSB-first: code j at bit w*j), then all the fp16 shifts, then
 * all the fp16 scales.  The section of (rung r, width index i = 0, 1, 2 for
 * w = 2, 4, 8) starts at byte section[3r + i]; it holds count[r] tokens x
 * nwidth[3r + i] groups.  Token t (rung rung[t]) is the rank[t]-th token of
 * its rung; group g is the slot[r*G + g]-th group of its width in rung r.
 * Every access is checked against `bytes`, the size of the storage buffer;
 * tokens whose rung lies outside the ladder, and groups with 0 bits, are
 * skipped. */
typedef struct dkv_wire {
  const int64_t* section; /* [rungs][3] */
  const int32_t* count;   /* [rungs] */
  const int32_t* rank;    /* [n] */
  const int16_t* slot;    /* [rungs][G] */
  const int16_t* nwidth;  /* [rungs][3] */
  int64_t bytes;
} dkv_wire_t;

/* codes u8 [n][G][64], shifts/scales f16 [n][G], rung [n] -> the storage
 * sections in `out` (scripts/kvtc_storage.py:63-75). */
int dkv_wire_pack(const uint8_t* codes, const uint16_t* low, const uint16_t* scale, const int16_t* rung, int32_t n,
                  dkv_ladder_t ladder, dkv_wire_t wire, uint8_t* out, void* stream);

/* The inverse (scripts/kvtc_storage.py:109-118, without the dequantize):
 * storage sections -> codes u8 [n][G][64], shifts/scales f16 [n][G].  Groups
 * that are skipped are left as the caller initialised them. */
int dkv_wire_unpack(const uint8_t* in, const int16_t* rung, int32_t n, dkv_ladder_t ladder, dkv_wire_t wire,
                    uint8_t* codes, uint16_t* low, uint16_t* scale, void* stream);

/* ---- K1: unpack + dequantize (replaces scripts/progressive.py:47-55
 *      dequantize applied to TokenStore rows at their hot prefix, :196-201;
 *      for ladder streams scripts/kvtc.py:62-79 quantize_groups' dequantized
 *      output, as read back by scripts/kvtc_storage.py:109-119) ----------
 * Tokens t0..t0+nt-1 of the stream -> out [nt][64G] in out_dtype.  With
 * DKV_F32 the values are bit-identical to the reference's fp32 dequantize
 * (and DKV_F16 to its fp16 cast of it). */
int dkv_unpack_dequant(const dkv_stream_t* s, int32_t t0, int32_t nt, void* out, int32_t out_dtype,
                       void* stream);

/* Encoder (replaces scripts/progressive.py:37-44 quantize8 and the error table
 * of :152-158): coefficients f32 [n][64G] -> codes u8 [n][G][64], low/span f16
 * [n][G] (bit-identical to the reference's fp32 arithmetic) and, unless
 * `errors` is NULL, errors f32 [n][G][9]: each group's squared error at 0..8
 * planes (fp32 sums over the 64 members, in this kernel's order). */
int dkv_quantize8(const float* coef, int32_t n, int32_t groups, uint8_t* codes, uint16_t* low, uint16_t* span,
                  float* errors, void* stream);

/* Centred token-matrix rows, the encoders' input to the PCA projection
 * (scripts/kvtc.py:137-140 to_matrix with :40-43 derotate and :50-53
 * token_matrix, then (matrix[start:end] - mean) as at :189 and
 * scripts/progressive.py:147-148): layer_ptrs is a device array of `layers`
 * device pointers to the per-layer caches [1][heads][tokens][head_dim] of
 * dtype DKV_F16 / DKV_BF16 / DKV_F32; out f32 [end-start][layers*heads*head_dim]
 * gets x - mean[f] with x de-rotated at its position (cos/sin f32
 * [tokens][head_dim]) for keys, or as is when cos and sin are NULL (values).
 * Bit-identical to that torch arithmetic (each operation rounded on its own). */
int dkv_centered_rows(const uint64_t* layer_ptrs, int32_t dtype, int32_t layers, int32_t heads, int32_t tokens,
                      int32_t head_dim, const float* cos, const float* sin, const float* mean, int32_t start,
                      int32_t end, float* out, void* stream);

/* Reference dequantize on unpacked codes (scripts/progressive.py:47-55):
 * codes u8 [n][G][64], low/span f16 [n][G], planes u8 [n or 1][G] -> f32 [n][64G]. */
int dkv_dequantize_codes(const uint8_t* codes, const uint16_t* low, const uint16_t* span, const uint8_t* planes,
                         int32_t planes_rows, int32_t n, int32_t groups, float* out, void* stream);

/* ---- bases ----------------------------------------------------------------
 * basis f32 [F][r] (columns = components, F = L*Hkv*d, row f = (l*Hkv+h)*d+dd;
 * scripts/kvtc.py:100-105, :88-97) -> the fp16 layouts the attention kernels
 * read:  key basis  [L][G][Hkv][d][64]  (per layer and 64-component group,
 *        every head's d x 64 block, components contiguous);
 *        value basis [L][Hkv][r][d]. */
int dkv_prepare_key_basis(const float* basis, int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t rank,
                          uint16_t* out, void* stream);
int dkv_prepare_value_basis(const float* basis, int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t rank,
                            uint16_t* out, void* stream);

/* ---- K2 + K3: one layer of attention over the codes ---------------------
 * Replaces scripts/compressed_attention.py:105-137 (CompressedContext._keys
 * and .attend): keys of the layer are rebuilt from the key codes on MFMA,
 * RoPE'd and scored without being written to memory; one softmax covers the
 * compressed tokens and the exact tokens; values are weighted in coefficient
 * space and the value basis is applied once per KV head.
 *
 * Sequences: `batch` conversations share the packed streams; sequence b owns
 * compressed tokens [cu_seqlens[b], cu_seqlens[b+1]) and exact tokens
 * [cu_exact[b], cu_exact[b+1]) (both int32 device arrays, batch+1 entries;
 * cu_seqlens_host mirrors cu_seqlens on the host to size the launch; with
 * batch == 1 the kernels take the lengths from the host mirrors, so a
 * captured graph replays with the lengths it was captured with). */
typedef struct dkv_attend_args {
  int32_t batch, q_len;
  int32_t layers, layer, kv_heads, head_dim, q_heads, rank;
  float scaling;
  dkv_stream_t key, value;
  const int32_t* cu_seqlens;      /* [batch+1] */
  const int32_t* cu_seqlens_host; /* host [batch+1] */
  const int32_t* positions;       /* [n_total] RoPE position of each compressed token, 0 .. rope_rows-1
                                     (the kernels clamp a position outside that range into it) */
  const uint16_t* key_basis;      /* fp16, dkv_prepare_key_basis layout */
  const uint16_t* value_basis;    /* fp16, dkv_prepare_value_basis layout */
  const float* mean_k;            /* [L][Hkv*d] */
  const float* mean_v;            /* [L][Hkv*d] */
  const float* rope_cos;          /* [P][d/2] f32 (first half of HF emb) */
  const float* rope_sin;          /* [P][d/2] */
  int32_t rope_rows;              /* P (> 0) */
  const void* query;              /* [batch][Hq][q_len][d], query_dtype */
  int32_t query_dtype;
  const int32_t* cu_exact;        /* [batch+1] with cu_exact[0] == 0, or NULL (no exact tokens) */
  const int32_t* cu_exact_host;   /* host mirror of cu_exact (<= 1024 exact tokens per sequence) */
  const void* key_exact;          /* [Hkv][E_total][d] in exact_dtype, RoPE applied */
  const void* value_exact;        /* [Hkv][E_total][d] in exact_dtype */
  const float* mask;              /* [q_len][E] additive (batch == 1 only) or NULL */
  void* out;                      /* [batch][q_len][Hq][d], out_dtype */
  int32_t out_dtype;
  int32_t exact_dtype;            /* DKV_F32 (0), DKV_F16 or DKV_BF16: the type of key_exact and value_exact
                                     (a model's own cache can be passed as it is; the kernels compute in f32);
                                     dkv_score_layer takes DKV_F32 only */
} dkv_attend_args_t;

size_t dkv_attend_workspace_bytes(const dkv_attend_args_t* a);

/* K1 for the attention kernels (replaces the per-conversation fp16
 * coefficient blocks of scripts/compressed_attention.py:71-77, built from
 * scripts/progressive.py:47-55 dequantize at each token's hot planes): decodes
 * every compressed token's key codes, truncated to min(planes, plane_cap)
 * bit-planes (8 = all hot planes; scoring "with the first 2 planes" passes 2),
 * into the workspace in the MFMA operand layout, and, when a->value.blob is
 * non-null, every token's value codes (all hot planes) with their affine
 * pairs for K3; a null value blob decodes the keys alone (question scoring
 * reads no values, and a score workspace has no room for them).  The decoded
 * codes depend on the streams only: call it
 * once before the layers of a decode step (and again after a stream
 * changes, e.g. dkv_gather_cold); every later dkv_attend_layer /
 * dkv_attend_scores / dkv_score_layer on the same workspace reads it.  Each
 * stream's table (pieces + 1 rows, or rungs) holds at most 4,096 rows
 * (DKV_ESHAPE otherwise). */
int dkv_attend_prepare(const dkv_attend_args_t* a, int32_t plane_cap, void* workspace, size_t workspace_bytes,
                       void* stream);
int dkv_attend_layer(const dkv_attend_args_t* a, void* workspace, size_t workspace_bytes, void* stream);

/* The two halves of dkv_attend_layer, in this order on one stream with the
 * same workspace: K2 (rebuild keys on MFMA, RoPE, score, per-tile softmax
 * statistics; replaces compressed_attention.py:105-126) and K3 (value
 * weighting in coefficient space, value basis once per KV head, exact-token
 * merge and normalisation; replaces :127-137).  Exposed so callers can time
 * or overlap them separately. */
int dkv_attend_scores(const dkv_attend_args_t* a, void* workspace, size_t workspace_bytes, void* stream);
int dkv_attend_values(const dkv_attend_args_t* a, void* workspace, size_t workspace_bytes, void* stream);

/* ---- K4a: question scoring over the hot tier ----------------------------
 * Replaces scripts/progressive.py:239-254 question_importance with
 * scripts/dimmer.py:52-66 scoring: for every layer, the attention each
 * compressed token receives from the q_len question tokens, summed over
 * query positions, the GQA group and the KV heads; the softmax spans the
 * compressed tokens, the exact tokens and the question's own keys (causal).
 * Uses the attend arguments (batch must be 1; out/value fields unused);
 * key_question is [Hkv][q_len][d] f32 (RoPE applied).  Call dkv_score_begin
 * once, then this for layers 0 .. layers-1 in order, on one workspace and
 * stream: each layer's contribution is added into importance [n] (f32) in
 * layer order, one call late (the call for layer l adds layer l-1's beside
 * computing layer l's softmax statistics), and the call for the last layer
 * adds its own too, so the vector is complete after that call. */
size_t dkv_score_workspace_bytes(const dkv_attend_args_t* a);
int dkv_score_begin(float* importance, int32_t n, void* stream);
int dkv_score_layer(const dkv_attend_args_t* a, const float* key_question, float* importance, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---- K4b: top-k (scripts/methods.py:246-247 importance[start:end].topk) --
 * Indices of the k largest values of scores [n] (ties: lower index first),
 * written in ascending index order to idx_out [k]. */
size_t dkv_topk_workspace_bytes(int32_t n);
int dkv_topk(const float* scores, int32_t n, int32_t k, int32_t* idx_out, void* workspace, size_t workspace_bytes,
             void* stream);

/* ---- allocation-free decode of one layer ---------------------------------
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation).  Does what dkv_attend_prepare(a, 8, ...) followed by
 * dkv_attend_layer(a, ...) do, with the workspace in a file-scope device array
 * of DKV_NOALLOC_MAX_BYTES that every GPU the library runs on holds until the
 * process ends; calls nothing that allocates.  A context whose workspace
 * (dkv_attend_workspace_bytes) exceeds the maximum is rejected with
 * DKV_EWORKSPACE before anything is launched.  Every call decodes the codes
 * again (the array keeps only the last call's contents); calls in sequence are
 * independent, calls that overlap on one GPU race.  The first call on a device
 * looks up that device's address of the array (hipGetSymbolAddress) and must
 * not be made under stream capture; later calls can be captured into a HIP
 * graph. */
#define DKV_NOALLOC_MAX_BYTES ((size_t)64 << 20)
int dkv_attend_layer_noalloc(const dkv_attend_args_t* a, void* stream);

/* ---- K4c: cold-plane gather (scripts/progressive.py:224-236 refine) ------
 * For the k selected tokens idx [k] (stream-local, distinct, each in 0..n-1:
 * one workgroup per entry repoints that token, so a repeated token races),
 * merge each token's hot
 * blob with its cold blob (cold + cold_tok_off[t]) into a full blob written
 * at refined + r*full_bytes (r = 0..k-1), then point the stream at it:
 * tok_off[t] = refined_base_off + r*full_bytes, pieces[t] = order.pieces.
 * `tok_off`/`pieces` are the stream's (mutable) arrays; `refined` must lie
 * inside the stream's blob allocation at byte offset refined_base_off. */
int dkv_gather_cold(const dkv_stream_t* s, const uint8_t* cold, const int64_t* cold_tok_off, const int32_t* idx,
                    int32_t k, uint8_t* refined, int64_t refined_base_off, int64_t* tok_off, int16_t* pieces,
                    void* stream);

/* ---- K4c for any token list, with the reference's byte count ------------
 * Replaces scripts/progressive.py:224-236 refine (the fetched count of :232
 * and the merge) for k tokens `rows` of a stream of n tokens that may repeat,
 * without a host round trip: fetched[0] += sum over the k entries as given of
 * full size - hot prefix of the token's pieces before the call (a repeated
 * token counts each time, as in the reference); each distinct token is merged
 * once, from its first entry r, into refined + r*full_bytes (so the refined
 * area must hold k full blobs); an entry outside 0..n-1 sets fetched[1] and
 * then no token is merged.  fetched[0..1] must be 0 on entry.  `owner` is an
 * int64 [n] array kept by the caller, zero at first: each call tags it with
 * `version`, which must be > 0 and grow from call to call on that array.
 * Calls that overlap on one owner array race. */
int dkv_refine_rows(const dkv_stream_t* s, int32_t n, const uint8_t* cold, const int64_t* cold_tok_off,
                    const int32_t* rows, int32_t k, uint8_t* refined, int64_t refined_base_off, int64_t* tok_off,
                    int16_t* pieces, int64_t* owner, int32_t version, int64_t* fetched, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DIMMERKV_H */
