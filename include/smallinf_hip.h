/*
 * smallinf_hip.h -- C ABI of the MI355X (gfx950) paged-attention decode path.
 *
 * One shared library, libsmallinf_hip.so, built with hipcc for gfx950. Every pointer argument is a device
 * pointer owned by the caller; the library allocates nothing on the device, keeps no pointer after a call
 * returns and launches asynchronously on the caller's stream (a hipStream_t passed as void*, NULL for the
 * default stream). No call synchronizes the host.
 *
 * Return codes: SIPA_OK (0) or a negative SIPA_E* code; sipa_last_error() then holds a message for the calling
 * thread. Shape, stride and dtype checks happen on the host before any launch, so a failed call launched nothing.
 *
 * Element strides are in elements of the tensor they describe, not bytes. Layouts follow the reference:
 *   KV pool, one layer: [H_kv, N, B, D] (head, block, offset in block, channel), each block row contiguous.
 *   A token's slot is block_table[p / B] * B + p % B; it addresses [:, block, offset] of every layer.
 */
#ifndef SMALLINF_HIP_H
#define SMALLINF_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIPA_ABI_VERSION 8

/* element types */
enum { SIPA_F32 = 0, SIPA_BF16 = 1, SIPA_F16 = 2, SIPA_I8 = 3 };

/* return codes */
enum {
  SIPA_OK = 0,
  SIPA_EINVAL = -1,       /* bad shape, stride, pointer or argument combination */
  SIPA_EUNSUPPORTED = -2, /* valid request outside the built support matrix */
  SIPA_EHIP = -3,         /* a HIP runtime call failed (launch, device query) */
  SIPA_EWORKSPACE = -4    /* workspace missing or smaller than sipa_decode_workspace_bytes() */
};

/* kv_mode of sipa_decode_params */
enum {
  SIPA_KV_PLAIN = 0,      /* K/V pools in q_dtype */
  SIPA_KV_INT8_TOKEN = 1, /* int8 K and V, one scale per (head, block, offset) each */
  SIPA_KV_INT8_KCHAN = 2  /* int8 K with one scale per (head, block, channel) and each sequence's partial last
                             block of K in a bf16 staging slot; int8 V with one scale per token */
};

/* impl of sipa_decode_params: AUTO picks MFMA where it applies, else the VALU fallback (any supported shape).
   VALU_STREAM / VALU_DOT2: the MFMA kernels' streaming structure with the dot products on the vector ALUs, fp32
   FMAs or v_dot2 pair products (bf16 q, block 16, head_dim 64/128, group 6-8, bf16 or int8 per-token pools); they
   exist to measure the matrix cores against the VALU and are never picked by AUTO. The bf16 MFMA kernel feeds P
   to its P.V product as a bf16 hi + lo pair (about 16 significant bits; the reference's TF32 P.V keeps 11);
   MFMA_PBF16 runs it with P rounded to one bf16 term (8 bits) instead, bf16 pools only, for measurement, never
   picked by AUTO. */
enum {
  SIPA_IMPL_AUTO = 0,
  SIPA_IMPL_VALU = 1,
  SIPA_IMPL_MFMA = 2,
  SIPA_IMPL_VALU_STREAM = 3,
  SIPA_IMPL_VALU_DOT2 = 4,
  SIPA_IMPL_MFMA_PBF16 = 5
};

/* combine of sipa_decode_params */
enum { SIPA_COMBINE_FUSED = 0, SIPA_COMBINE_KERNEL = 1 };

/*
 * Paged decode attention: one query token per sequence over its paged context.
 *   out[s, h*G + g, :] = sum_{t < ctx[s]} softmax_t(scale * q[s, h*G+g, :] . k_t) v_t,   G = Hq / Hkv,
 *   k_t, v_t = pool[h, block_tables[s, t / B], t % B, :].
 * Replaces paged_decode_attention / _decode_kernel / _combine_kernel (reference engine/triton_decode.py:51-161,
 * 188-238).
 */
typedef struct sipa_decode_params {
  int32_t struct_size;   /* sizeof(sipa_decode_params) of this ABI: guards against a stale binding */
  int32_t num_seqs;      /* S */
  int32_t num_q_heads;   /* Hq */
  int32_t num_kv_heads;  /* Hkv; Hq % Hkv == 0 */
  int32_t head_dim;      /* D */
  int32_t block_size;    /* B; 64 % B == 0 (reference engine/triton_decode.py:211) */
  int32_t num_blocks;    /* N, blocks in the pool */
  int32_t max_context;   /* max(context_lens), known on the host; sizes the split grid */
  int32_t num_splits;    /* <= 0: choose from the device's CU count (sipa_choose_splits) */
  int32_t q_dtype;       /* SIPA_F32 or SIPA_BF16: q, out, and the pool when kv_mode == SIPA_KV_PLAIN */
  int32_t kv_mode;       /* SIPA_KV_* */
  int32_t impl;          /* SIPA_IMPL_* */
  int32_t combine;       /* SIPA_COMBINE_* */
  float scale;           /* softmax scale, head_dim^-0.5 in the model; positive and finite (else SIPA_EINVAL) */
  const void* q;         /* [S, Hq, D]; last dim contiguous */
  int64_t q_stride_s, q_stride_h;
  const void* k_cache;   /* [Hkv, N, B, D] */
  const void* v_cache;   /* [Hkv, N, B, D] */
  int64_t kv_stride_h, kv_stride_n; /* block rows are contiguous: offset stride D, channel stride 1 */
  const int32_t* block_tables; /* [S, bt_width]; entries past a sequence's context (up to ceil(max_context / B))
                                  may be loaded but are never used; ids are clamped to [0, num_blocks) */
  int64_t bt_stride_s;
  const int32_t* context_lens; /* [S], each >= 1, the new token included; clamped to max_context */
  void* out;             /* [S, Hq, D] in q_dtype */
  int64_t out_stride_s, out_stride_h;
  /* SIPA_KV_INT8_TOKEN: k_scale, v_scale [Hkv, N, B].  SIPA_KV_INT8_KCHAN: k_scale [Hkv, N, D] (a zero block
     stride gives one scale per (head, channel) for the whole pool), v_scale [Hkv, N, B]. SIPA_F16 or SIPA_F32. */
  const void* k_scale;
  int32_t k_scale_dtype;
  int64_t ks_stride_h, ks_stride_n;
  const void* v_scale;
  int32_t v_scale_dtype;
  int64_t vs_stride_h, vs_stride_n;
  /* SIPA_KV_INT8_KCHAN only: bf16 staging [Hkv, num_stage, B, D] and the staging slot of each sequence's partial
     last block (-1 when ctx % B == 0); slots past num_stage - 1 are clamped to it (wrong results, no access
     outside the staging pool). */
  const void* stage;
  int64_t st_stride_h, st_stride_n, st_stride_b;
  const int32_t* tail_slots;
  /* Split partials and merge counters; at least sipa_decode_workspace_bytes() bytes, 256-byte aligned. The
     first 256 KiB hold the merge counters (at most 65536 (sequence, KV head) pairs per split call), which must be
     zero before the first call that uses the buffer; every completed call leaves them zero again and no call
     writes partials there, so one buffer serves decode and prefill calls of any size. Calls that share one
     workspace must be ordered (one stream). May be NULL when 1 split runs. */
  void* workspace;
  int64_t workspace_bytes;
  /* Optional work list: num_items > 0 launches one workgroup
     per item instead of the (sequence, KV head, split) grid. Items are 8 int32 each, 16-byte aligned, in device
     memory: {seq, kv_head, split, splits_of_pair, start, end, 0, 0}, the pair's tokens [start, end) and its
     splits numbered 0 .. splits_of_pair - 1. num_splits must be the largest splits_of_pair (it sizes the
     workspace); splits are always merged by the last-arriving workgroup. Built by sipa_build_work_list from the
     host-side context lengths (sipa_check_work_list validates a list built elsewhere). A list that does not match
     context_lens gives wrong results (every access stays in bounds); a list inconsistent with itself (a pair
     with more or fewer items than its splits_of_pair) also leaves that pair's merge counter non-zero, and every
     later call on the same workspace then merges wrongly until the counter region is zeroed again. */
  const int32_t* work_items;
  int32_t num_items;
  int32_t bt_width;      /* entries per block_tables row; must be >= ceil(max_context / B) (SIPA_EINVAL otherwise) */
  int32_t num_stage;     /* SIPA_KV_INT8_KCHAN: staging slots in stage (>= 1); ignored by the other modes */
} sipa_decode_params;

int32_t sipa_abi_version(void);
const char* sipa_last_error(void);

/* Compute units of a device (256 on MI355X); < 0 on error. */
int32_t sipa_device_cu_count(int32_t device);

/*
 * Splits per sequence for a call over bf16/fp32 pools. Replaces the reference's 20-SM policy choose_splits
 * (reference engine/triton_decode.py:164-172) with one sized from the CU count: at most one (sequence, KV head,
 * split) workgroup per CU, ceil(cu_count / (num_seqs * num_kv_heads)) splits, but no split under 512 tokens of
 * max_context past 8 splits (short contexts: up to 8 splits of at least 128 tokens), and none over 2048 (so a
 * long sequence in a full grid is spread over several CUs).
 */
int32_t sipa_choose_splits(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context, int32_t cu_count);

/*
 * The split count sipa_decode uses when num_splits <= 0, for pools of kv_mode (SIPA_KV_*): sipa_choose_splits
 * for bf16/fp32 pools; for INT8 pools, whose kernels run two workgroups per CU, twice the CUs, splits of at
 * least 256 tokens past 8 splits, and at least ceil(max_context / 4096) (INT8 calls use that many whatever num_splits asks:
 * size the workspace for the larger count). cu_count <= 0: the current device's. No counterpart in the
 * reference (its one policy serves every mode).
 */
int32_t sipa_choose_splits_for(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context, int32_t cu_count,
                               int32_t kv_mode);

/* Tokens per split for a call with num_splits splits: ceil(max_context / num_splits) rounded up to a multiple
 * of 64 tokens, at most 32768. Calls launch ceil(max_context / chunk) splits, which may be fewer than asked. */
int32_t sipa_split_chunk(int32_t max_context, int32_t num_splits);

/* The split grid sipa_decode launches for a call of these sizes without a work list, on the MFMA kernels (bf16
 * query, 16-token blocks, head_dim 64 / 128): returns the number of splits per sequence and writes the token counts
 * of its splits: the first *n_old splits hold *chunk_old tokens, the others *chunk (*n_old 0: all *chunk). INT8
 * per-channel-K pools on a grid of exactly two workgroups per CU take two lengths (the earlier-dispatched workgroup
 * of each CU's pair streams faster and gets the longer split). Replaces the chunk computation of the reference's
 * wrapper (engine/triton_decode.py:203-204). Negative SIPA_E* on bad arguments. */
int32_t sipa_decode_split_grid(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context, int32_t num_splits,
                               int32_t kv_mode, int32_t* chunk, int32_t* chunk_old, int32_t* n_old);

/* Workspace bytes sipa_decode needs for these sizes (0 when num_splits resolves to 1). */
int64_t sipa_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t num_splits);

int32_t sipa_decode(const sipa_decode_params* p, void* stream);

/*
 * sipa_decode without a caller-supplied workspace, for callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc. No counterpart in the reference. The same
 * kernels and launches as sipa_decode (identical results for identical parameters); p->workspace and
 * p->workspace_bytes are ignored. The split partials and merge counters live in a 16 MiB device array inside the
 * library (one per GPU, held until the process ends; the first call on a GPU also launches one small kernel that
 * zeroes its counters). A call whose splits need more than that (sipa_decode_workspace_bytes() > 16 MiB) fails with
 * SIPA_EWORKSPACE before launching anything. Allocates nothing: no hipMalloc, hipFree or allocating library call.
 * Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU (different streams, or
 * threads) race and give wrong results; order them on one stream. Each completed call leaves the array's merge
 * counters at zero, which the next call relies on; a call that did not complete (an aborted launch) or a work list
 * that disagrees with the context lengths can leave one non-zero, and later calls would then merge that pair
 * wrongly. The recovery is sipa_decode_noalloc_reset.
 */
int32_t sipa_decode_noalloc(const sipa_decode_params* p, void* stream);

/*
 * Zeroes the merge counters of the current GPU's sipa_decode_noalloc array with one small kernel on `stream`
 * (no memset node, so it may be captured in a HIP graph), after which calls merge correctly again. Ordered like a
 * call: enqueue it where no sipa_decode_noalloc call on that GPU is in flight. Allocates nothing. No counterpart in
 * the reference; for the callers of sipa_decode_noalloc.
 */
int32_t sipa_decode_noalloc_reset(void* stream);

/*
 * Paged attention for multi-token rows (prefill chunks): replaces the reference's gather path for rows with
 * several new tokens (reference engine/paged_cache.py:149-155,174-175 with engine/attention.py:6-28). For each
 * sequence s, rows query_starts[s] .. query_starts[s] + query_lens[s] - 1 of q are its new tokens at positions
 * context_lens[s] - query_lens[s] .. context_lens[s] - 1 (their K/V already written to the pool); each attends
 * causally to positions 0 .. its own, query head g to KV head g / (Hq / Hkv), softmax in fp32 with the
 * probabilities rounded to bf16 for P.V, written to the same rows of out. bf16 q and out, bf16 or INT8 pools;
 * 16-token blocks; head_dim 64 or 128; group Hq / Hkv <= 8; max_context <= 32768. Context lengths are clamped to max_context and
 * block ids to [0, num_blocks); q and out rows must be 16-byte aligned.
 */
typedef struct sipa_prefill_params {
  int32_t struct_size;   /* sizeof(sipa_prefill_params) */
  int32_t num_seqs;
  int32_t num_tokens;    /* T: rows of q and out (rows past T are neither read nor written) */
  int32_t num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_context;
  int32_t max_query_len; /* max over s of query_lens[s] (sizes the grid) */
  float scale;           /* softmax scale; positive and finite (else SIPA_EINVAL) */
  const void* q;         /* [T, Hq, D] bf16, last dim contiguous */
  int64_t q_stride_t, q_stride_h;
  const void* k_cache;   /* [Hkv, N, B, D] bf16 */
  const void* v_cache;
  int64_t kv_stride_h, kv_stride_n;
  const int32_t* block_tables; /* [S, bt_width]; a sequence's first ceil(context / B) entries are read */
  int64_t bt_stride_s;
  const int32_t* context_lens; /* [S] tokens in the cache, this forward's included */
  const int32_t* query_starts; /* [S] first row of each sequence's new tokens */
  const int32_t* query_lens;   /* [S] new tokens of each sequence (>= 1) */
  void* out;                   /* [T, Hq, D] bf16 */
  int64_t out_stride_t, out_stride_h;
  /* SIPA_KV_PLAIN: bf16 pools. SIPA_KV_INT8_TOKEN / SIPA_KV_INT8_KCHAN: int8 pools with scales and (format B)
     staging laid out as in sipa_decode_params; K/V are dequantized as the reference's gather path does,
     q * s in fp32 rounded to bf16, with format B's keys past the last full block taken from the staging slot. */
  int32_t kv_mode;
  const void* k_scale;
  int32_t k_scale_dtype;
  int64_t ks_stride_h, ks_stride_n;
  const void* v_scale;
  int32_t v_scale_dtype;
  int64_t vs_stride_h, vs_stride_n;
  const void* stage;            /* [Hkv, num_stage, B, D] bf16 */
  int64_t st_stride_h, st_stride_n, st_stride_b;
  int32_t num_stage;
  const int32_t* tail_slots;   /* [S] staging slot of each sequence's partial last block, -1 if none (slots are
                                  clamped to [0, num_stage)) */
  /* Key splits per 16-token query tile (<= 0: sipa_prefill_splits with units = S x Hkv x query tiles) and the
     workspace they need when more than one split runs: sipa_prefill_workspace_bytes() bytes, laid out and reused
     as sipa_decode_params.workspace (the same buffer may serve both); at most 65536 KV heads x query tiles. */
  int32_t num_splits;
  void* workspace;
  int64_t workspace_bytes;
  int32_t bt_width;             /* entries per block_tables row; must be >= ceil(max_context / 16) */
  /* Split merge (ABI 4): SIPA_MERGE_AUTO reads a unit's partials from the L2 of the XCD its splits ran on when
     they all shared one (the kernel places them so), through memory otherwise; SIPA_MERGE_MEMORY always reads
     them through memory (agent-coherent loads). Both give the same bits. */
  int32_t merge_path;
  /* Workgroup layout (ABI 6), a SIPA_PREFILL_* value. A column tile is a query head and 16 of a unit's tokens.
     SIPA_PREFILL_AUTO lets the library choose from g8, the grid of 8-column workgroups: SIPA_PREFILL_W8X1 for
     g8 <= CUs; for a chunk at least its own length into its context, SIPA_PREFILL_W16H2 over bf16 pools with 8
     or more key splits of at most 1024 keys, else SIPA_PREFILL_W16X1 with one split or splits of at least 1024
     keys, else W8X1; for fresh prompts W8X1 up to 3 workgroups per CU, then W16X1, except SIPA_PREFILL_W4X2
     beyond 4 per CU at head_dim 64. Format B pools (SIPA_KV_INT8_KCHAN) take W4X2 (W4X2 or W8X1 when forced). W4X2 and
     W8X1 give the same bits; W16X1 too with one split (with several, a row may go through the split merge's
     fp16 partials in one layout and not in the other); W16H2 combines key splits in its own order. Every
     layout meets the same error bound. With W16H2, num_splits counts key chunks, two to a workgroup. */
  int32_t wg_layout;
} sipa_prefill_params;

enum { SIPA_MERGE_AUTO = 0, SIPA_MERGE_MEMORY = 1 };
enum {
  SIPA_PREFILL_AUTO = 0,
  SIPA_PREFILL_W4X2 = 1,  /* 4 waves of two column tiles: 8 column tiles per workgroup */
  SIPA_PREFILL_W8X1 = 2,  /* 8 waves of one column tile: 8 column tiles per workgroup */
  SIPA_PREFILL_W16X1 = 3, /* 16 waves of one column tile: 16 column tiles (a unit of twice the tokens) */
  SIPA_PREFILL_W16H2 = 4  /* 16 waves: 8 column tiles, each over two consecutive key splits combined in the
                             workgroup (half the workgroups per unit) */
};

int32_t sipa_prefill(const sipa_prefill_params* p, void* stream);

/* Key splits for a prefill call (no counterpart in the reference, whose gather path has no grid): about two
 * workgroups per CU over the call's 8-column units, at least 256 keys per split, at most 32 splits. An 8-column
 * unit is a KV head and 16 tt new tokens of one sequence, tt = 8 / G 16-token subtiles (at least 1) for a group
 * of G = Hq / Hkv query heads (head_dim is part of the policy's signature and does not change it today);
 * query_tiles = sum over sequences of ceil(query_len / 16). A 16-column layout keeps the split count and runs
 * half as many units. cu_count <= 0 asks the current device. */
int32_t sipa_prefill_splits(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int64_t query_tiles,
                            int32_t max_context, int32_t cu_count);

/* Workspace bytes sipa_prefill needs for these sizes and num_splits under any workgroup layout (0 when one
 * split runs). */
int64_t sipa_prefill_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                                     int32_t head_dim, int32_t max_query_len, int32_t max_context,
                                     int32_t num_splits);

/*
 * Work list for a ragged batch (no counterpart in the reference, whose grid is always (sequence, KV head,
 * split)): every (sequence, KV head) pair is cut into ceil(ctx / piece) splits of near-equal length, piece about
 * sum(ctx) * num_kv_heads / (cu_count * items_per_cu) tokens (a multiple of 64, at most max_piece; max_piece <= 0
 * means 32768, and INT8 pools need max_piece <= 4096), and the items are ordered longest first, so the longest
 * work starts first and consecutive workgroups spread over the XCDs. Pieces are at least 512 tokens (a small
 * batch's long sequence is not cut into more merges than its streaming saves), or 256 when max_piece <= 4096:
 * the INT8 kernels, two workgroups per CU, do better with the shorter pieces.
 * context_lens_host [num_seqs] (each >= 1) are the lengths the decode call will read. Writes at most capacity
 * items (8 int32 each) to items_out and the largest split count of a pair to *max_splits; returns the number of
 * items, or a negative SIPA_E* code (items_out may be NULL to ask for the count).
 */
int32_t sipa_build_work_list(const int32_t* context_lens_host, int32_t num_seqs, int32_t num_kv_heads,
                             int32_t cu_count, int32_t items_per_cu, int32_t max_piece, int32_t* items_out,
                             int32_t capacity, int32_t* max_splits);

/*
 * Checks a host copy of a work list before it is uploaded (no counterpart in the reference): every item's
 * sequence and KV head in range, each pair's items numbered 0 .. splits_of_pair - 1 exactly once with the same
 * splits_of_pair, their token ranges [start, end) within [0, max_context), in order and without overlap, and
 * no split count above num_splits. Returns SIPA_OK or SIPA_EINVAL (sipa_last_error() names the first bad item).
 * Lists from sipa_build_work_list always pass.
 */
int32_t sipa_check_work_list(const int32_t* items_host, int32_t num_items, int32_t num_seqs, int32_t num_kv_heads,
                             int32_t max_context, int32_t num_splits);

/*
 * Per-forward packed metadata on the device (the device-side form of reference engine/paged_cache.py:55-90,
 * build_metadata, with the slot rule of engine/block_manager.py:118-123). tables [table_rows, table_stride] int32
 * hold each live sequence's block table in one row (maintained by the caller); seq_info [3 S + 1] int32 is the
 * forward's rows[S] (table row of each sequence), starts[S] (position of its first new token) and query_starts
 * [S + 1] (cumulative new-token counts, query_starts[S] = num_tokens). Writes, for every token t,
 * positions[t] = starts[s] + t - query_starts[s], slots[t] = table[row][p / B] * B + p % B, slot_blocks[t],
 * slot_offsets[t]; for every sequence, context_lens[s] = starts[s] + its new tokens, last_rows[s] =
 * query_starts[s + 1] - 1 and block_tables[s, :out_width] = its first ceil(context / B) table entries, then -1.
 * Table indices are clamped to the table, so malformed rows read wrong entries, never outside it.
 */
int32_t sipa_paged_metadata(const int32_t* tables, int64_t table_stride, int32_t table_rows, int32_t table_width,
                            const int32_t* seq_info, int32_t num_seqs, int32_t num_tokens, int32_t block_size,
                            int32_t out_width, int64_t* positions, int64_t* slots, int64_t* slot_blocks,
                            int64_t* slot_offsets, int64_t* last_rows, int32_t* block_tables,
                            int32_t* context_lens, void* stream);

/*
 * The five store entry points below use their indices as given, as the reference's store kernels and index_put
 * stores do with valid input: blocks and dst in [0, N), offsets in [0, B), src in [0, n_src), rows in [0, T).
 * The caches derive them from the block manager's slots; a caller with indices of unknown origin checks them
 * first (the decode and prefill kernels, which only read, clamp theirs instead).
 */

/*
 * Per-token INT8 quantize-and-store (reference engine/triton_quant.py:24-39,61-71 and the quantizer
 * engine/quant.py:22-31): for every (t, h),
 *   s = fp16(max_d |x[t,h,d]| / 127);  q[d] = s > 0 ? clamp(rint(x[t,h,d] / float(s)), -127, 127) : 0
 * with IEEE fp32 division and round-half-even, stored to q_pool[h, blocks[t], offsets[t], :] (int8) and
 * s_pool[h, blocks[t], offsets[t]] (fp16).
 *   x [T, H, D] in x_dtype (SIPA_F32 / SIPA_BF16 / SIPA_F16), last dim contiguous;
 *   blocks, offsets [T] int64; q_pool [H, N, B, D] int8 (offset stride D); s_pool [H, N, B] fp16.
 */
int32_t sipa_quantize_store_tokens(const void* x, int32_t x_dtype, int64_t x_stride_t, int64_t x_stride_h,
                                   int32_t T, int32_t H, int32_t D, const int64_t* blocks,
                                   const int64_t* offsets, int8_t* q_pool, int64_t q_stride_h,
                                   int64_t q_stride_n, int32_t B, void* s_pool, int64_t s_stride_h,
                                   int64_t s_stride_n, void* stream);

/*
 * Two sipa_quantize_store_tokens calls in one launch, with no reference counterpart (the reference's cache
 * makes the two calls, engine/quant_cache.py:161-163): x -> (q_pool, s_pool) and x2 -> (q_pool2, s_pool2) at the
 * same (blocks[t], offsets[t]), x2 with its own row and head strides, the second pools with the first's strides.
 * For the per-token format's V and K of one layer. Results equal the two separate calls bit for bit.
 */
int32_t sipa_quantize_store_tokens_kv(const void* x, const void* x2, int32_t x_dtype, int64_t x_stride_t,
                                      int64_t x_stride_h, int64_t x2_stride_t, int64_t x2_stride_h, int32_t T,
                                      int32_t H, int32_t D, const int64_t* blocks, const int64_t* offsets,
                                      int8_t* q_pool, int8_t* q_pool2, int64_t q_stride_h, int64_t q_stride_n,
                                      int32_t B, void* s_pool, void* s_pool2, int64_t s_stride_h,
                                      int64_t s_stride_n, void* stream);

/*
 * Per-channel INT8 quantize-and-store of whole blocks (reference engine/triton_quant.py:42-58,74-84): for every
 * (i, h) the [B, D] tile src_pool[h, src[i]] gets one scale per channel over its B tokens,
 *   s[d] = fp16(max_b |x[b,d]| / 127), codes as above, stored to q_pool[h, dst[i]] and s_pool[h, dst[i], :].
 *   src_pool [H, n_src, B, D] in src_dtype (bf16 staging in the cache); src, dst [n] int64;
 *   q_pool [H, N, B, D] int8; s_pool [H, N, D] fp16.
 */
int32_t sipa_quantize_store_blocks(const void* src_pool, int32_t src_dtype, int64_t src_stride_h,
                                   int64_t src_stride_n, int64_t src_stride_b, const int64_t* src,
                                   const int64_t* dst, int32_t n, int32_t H, int32_t B, int32_t D,
                                   int8_t* q_pool, int64_t q_stride_h, int64_t q_stride_n, void* s_pool,
                                   int64_t s_stride_h, int64_t s_stride_n, void* stream);

/*
 * The same per-channel block quantization with the block's B tokens taken from rows of x [T, H, D]:
 * block i holds rows[i*B + b], b < B. Each value is rounded to bf16 first, as the reference's cache does for
 * blocks one forward writes whole (reference engine/quant_cache.py:147-153,171-177).
 */
int32_t sipa_quantize_store_block_rows(const void* x, int32_t x_dtype, int64_t x_stride_t, int64_t x_stride_h,
                                       const int64_t* rows, const int64_t* dst, int32_t n, int32_t H,
                                       int32_t B, int32_t D, int8_t* q_pool, int64_t q_stride_h,
                                       int64_t q_stride_n, void* s_pool, int64_t s_stride_h,
                                       int64_t s_stride_n, void* stream);

/*
 * Scatter-store of token vectors into a pool (reference engine/paged_cache.py:135-139 for the K/V pool and
 * engine/quant_cache.py:139-141,165-167 for the bf16 staging slots):
 *   pool[h, blocks[i], offsets[i], :] = convert(x[rows ? rows[i] : i, h, :])   for i < n, h < H.
 * x in x_dtype, pool in pool_dtype (SIPA_F32 / SIPA_BF16 / SIPA_F16; conversion rounds to nearest even).
 * A second tensor pair (x2, pool2) with the same shapes and dtypes (x2 with its own row and head strides, pool2
 * with pool's strides) is stored in the same launch when x2 != NULL.
 */
int32_t sipa_store_tokens(const void* x, const void* x2, int32_t x_dtype, int64_t x_stride_t,
                          int64_t x_stride_h, int64_t x2_stride_t, int64_t x2_stride_h, const int64_t* rows,
                          int32_t n, int32_t H, int32_t D,
                          const int64_t* blocks, const int64_t* offsets, void* pool, void* pool2,
                          int32_t pool_dtype, int64_t p_stride_h, int64_t p_stride_n, int64_t p_stride_b,
                          void* stream);

/*
 * Format B ("int8-kchannel") writes of a decode step in one launch, with no reference counterpart (the reference's
 * cache makes three calls, engine/quant_cache.py:161-170, and this library's three equivalents are
 * sipa_quantize_store_tokens, sipa_store_tokens and sipa_quantize_store_blocks). For every row t < T (one new
 * token):
 *   1. v[t] quantized per token into v_pool[h, blocks[t], offsets[t], :] and v_scale[h, blocks[t], offsets[t]];
 *   2. the bf16 rounding of k[t] stored to stage[h, stage_slots[t], offsets[t], :];
 *   3. when quant_dst[t] >= 0 (quant_dst == NULL: when offsets[t] == B - 1, into blocks[t]), the slot's B tokens
 *      (row t's just staged) quantized per channel into k_pool[h, quant_dst[t]] and k_scale[h, quant_dst[t], :].
 * Results equal those three calls bit for bit when no two rows share a staging slot (a decode step: one row per
 * sequence). Rows that do share one (the graph runner's padding rows, all on a scratch block) leave that slot
 * and its destination with unspecified contents.
 *   k, v [T, H, D] in x_dtype (SIPA_F32 / SIPA_BF16 / SIPA_F16), last dim contiguous; blocks, offsets,
 *   stage_slots, quant_dst [T] int64; v_pool, k_pool [H, N, B, D] int8 (offset stride D); v_scale [H, N, B] and
 *   k_scale [H, N, D] fp16; stage [H, n_stage, B, D] bf16.
 */
typedef struct sipa_kchan_write_params {
  const void* k;
  const void* v;
  int32_t x_dtype;
  int64_t k_stride_t, k_stride_h, v_stride_t, v_stride_h;
  int32_t T, H, D, B;
  const int64_t* blocks;
  const int64_t* offsets;
  const int64_t* stage_slots;
  const int64_t* quant_dst; /* may be NULL */
  int8_t* v_pool;
  void* v_scale;
  int8_t* k_pool;
  void* k_scale;
  int64_t q_stride_h, q_stride_n;   /* both int8 pools */
  int64_t vs_stride_h, vs_stride_n; /* v_scale */
  int64_t ks_stride_h, ks_stride_n; /* k_scale */
  void* stage;
  int64_t st_stride_h, st_stride_n, st_stride_b;
} sipa_kchan_write_params;

int32_t sipa_kchan_write_rows(const sipa_kchan_write_params* p, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SMALLINF_HIP_H */
