// Paged attention for multi-token rows (prefill chunks) on the matrix cores (gfx950).
//
// Reference: the reference serves these rows with its gather path (engine/paged_cache.py:149-155,174-175):
// every sequence's K/V are copied out of the pool and engine/attention.py:6-28 computes causal GQA attention
// (query at position p sees keys 0 .. p, query head g uses KV head g / G, softmax in fp32, probabilities rounded
// to the model dtype before P.V). This kernel computes the same rows in place from the pool.
//
// Work unit: (sequence s, KV head h, 16 tt consecutive new tokens). The unit's keys are positions [0, P0 + ntok)
// of the sequence, P0 the position of the unit's first token; they are cut into splits of `chunk` keys, one
// workgroup each, so that a short chunk over a long context still fills the chip. The four waves of a workgroup
// stream the same key tiles (64 keys at head_dim 64, 32 at 128), which the workgroup loads cooperatively into
// double-buffered LDS (one HBM read per split), and each wave owns its own column tiles (a query head and 16 of
// the unit's tokens), so no cross-wave merge is needed. A unit with one split writes its rows; otherwise every
// split writes its softmax state (m, l, unnormalised O) and the last split workgroup of the unit to finish merges
// them, as the decode kernels do.
// Per tile and head, with the decode kernels' layouts (decode.hip) and the query tokens in place of the heads:
//   S^T[16 keys x 16 tokens] = K[16 x 32 d] . Q^T[32 d x 16 tokens]     v_mfma_f32_16x16x32_bf16
//   causal mask: key position > token position -> -inf; online softmax per token (exp2 domain, lazy rescale)
//   O^T[16 d x 16 tokens] += V^T . P^T   (V^T by transposing LDS reads, P^T from the S^T registers)
#include <algorithm>
#include <type_traits>

#include "decode_common.h"

namespace sipa {

struct PrefillArgs {
  const void* q;
  int64_t q_st, q_sh;
  const void* k;
  const void* v;
  int64_t kv_sh, kv_sn;
  const int32_t* bt;
  int64_t bt_ss;
  int32_t bt_w;  // entries per table row (>= ceil(max_ctx / 16)): columns are clamped below it
  const int32_t* ctx;     // [S] context lengths after this forward's writes
  const int32_t* qstart;  // [S] first row of each sequence's new tokens in q / out
  const int32_t* qlen;    // [S] new tokens per sequence
  void* out;
  int64_t o_st, o_sh;
  int32_t S, G, qtiles;   // qtiles = ceil(max new tokens / (16 tt))
  int32_t npair;           // S * Hkv
  int32_t tt;              // 16-token subtiles per unit: G * tt <= 8 column tiles
  int32_t T, nb, max_ctx;  // rows of q / out, pool blocks, context clamp
  int32_t nsplit, chunk;   // key splits per unit, keys per split (a multiple of 64)
  // INT8 pools (kernel MODE 1, 2): scales and format B's staging, as in sipa_prefill_params
  const void* ks;
  const void* vs;
  bool ks_f32, vs_f32;
  bool ks_vec;  // MODE 2: each block's channel-scale row is 16-byte aligned (vector loads of 16 scales)
  int64_t ks_sh, ks_sn, vs_sh, vs_sn;
  const uint16_t* stage;
  int64_t st_sh, st_sn, st_sb;
  int32_t n_stage;
  const int32_t* tails;
  float scale_log2;
  bool mem_merge;          // merge every unit through memory (SIPA_MERGE_MEMORY)
  int* counters;           // [units] split arrivals, zero between launches
  float* pm;               // [units][nsplit][8 columns][16 tokens] running max (exp2 domain)
  float* pl;               // same shape: softmax denominators, the row's exponent e in the low 8 mantissa bits
  float* part;             // [units][nsplit][8 columns][16 tokens][D] each split's output O / l 2^-e, as fp16
};

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Workgroup layouts: NC column tiles (a query head and 16 tokens) per workgroup, CW per wave, NC / CW waves.
//   SIPA_PREFILL_W4X2 (NC 8, CW 2): 4 waves; each K/V operand read serves two column tiles. Large grids.
//   SIPA_PREFILL_W8X1 (NC 8, CW 1): 8 waves, twice the waves per CU for grids of at most 2 workgroups per CU.
//   SIPA_PREFILL_W16X1 (NC 16, CW 1): 16 waves over two query tiles' worth of columns, one workgroup per CU where
//   two 8-column workgroups would share it (the later-dispatched of two co-resident workgroups ran 30% longer
//   than the first, its solo tail idling the CU's other SIMD slots); each K/V tile load serves both query tiles.
// Four column tiles per wave (at head_dim 64) measured slower, 86.7 -> 112 us on four 2048-token prompts, with
// the register use halving the waves per SIMD and the 32-token units coarsening the causal tiles.
constexpr int kPrefillMaxGroup = 8;
struct PfShape {
  int nc, cw, kh;
};
static inline PfShape prefill_shape(int layout) {
  switch (layout) {
    case SIPA_PREFILL_W8X1: return PfShape{8, 1, 1};
    case SIPA_PREFILL_W16X1: return PfShape{16, 1, 1};
    case SIPA_PREFILL_W16H2: return PfShape{8, 1, 2};
    default: return PfShape{8, 2, 1};
  }
}

// 16-token subtiles per unit for a GQA group of G heads: as many as fit the workgroup's NC column tiles (NC 8:
// G = 7: 1, G = 4: 2, G = 1: 8), so every group size keeps the waves busy.
static inline int prefill_subtiles(int G, int nc) { return G >= nc ? 1 : nc / G; }
constexpr int kPrefillMaxSplits = 32;


template <int D>
struct PrefillSmem {  // one 32-key row group; a KT-key tile is KT / 32 of them
  // bf16 per LDS row of a 32-key tile. D + 16 keeps the waves' K (16-byte rows) and transposing V reads free
  // of bank conflicts; at D + 8 46% of the LDS's active cycles were conflicts, which cost little while two column
  // tiles per wave shared each read but 1.5 us of a 512-token chunk at 8K (3.5 at head_dim 128) with one.
  static constexpr int kPitch = D + 16;
  static constexpr int kTile = 32 * kPitch;  // elements of one K or V tile
};

// A cooperative-load chunk as it arrives from memory, per pool format: MODE 0 bf16 K/V, 8 channels of one key
// (16 bytes each); MODE 1 int8 codes, 16 channels of one key (16 bytes each), with per-token K and V scales;
// MODE 2 the same codes with the block's 16 K channel scales (fp16: two 16-byte words, fp32: four), the token's
// V scale, and the bf16 staged K of the sequence's partial last block (used when `staged`). Scales are kept as
// raw fp16 or fp32 bits until the LDS store, so that their loads are waited for only there.
template <int MODE>
struct KvRaw;
template <>
struct KvRaw<0> {
  u32x4 k, v;
};
template <>
struct KvRaw<1> {
  u32x4 k, v;
  uint32_t ks, vs;
};
template <>
struct KvRaw<2> {
  u32x4 k, v;
  u32x4 ks[4];
  uint32_t vs;
  u32x4 st[2];
  bool staged;
};

// Channel scale j (0 .. 15) of a chunk from its raw words: fp16 bits packed two per dword, or fp32 bits.
__device__ __forceinline__ float chan_scale(const u32x4 (&w)[4], bool f32, int j) {
  if (f32) return __uint_as_float(w[j >> 2][j & 3]);
  const uint32_t d = w[j >> 3][(j >> 1) & 3];
  return f16_bits_to_f32((j & 1) ? d >> 16 : d & 0xffffu);
}

__device__ __forceinline__ uint32_t scale_bits(const void* base, bool f32, int64_t i) {
  return f32 ? ((const uint32_t*)base)[i] : (uint32_t)((const uint16_t*)base)[i];
}

__device__ __forceinline__ float scale_value(uint32_t bits, bool f32) {
  return f32 ? __uint_as_float(bits) : f16_bits_to_f32(bits);
}

// 8 int8 codes -> 8 bf16 of code * scale(j), computed in fp32 and rounded to nearest even (the reference's
// dequantize(q, s, bf16): (q.float() * s.float()).to(bfloat16)).
template <typename Scale>
__device__ __forceinline__ u32x4 dequant8(u32x2 codes, Scale scale) {
  u32x4 out;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const uint32_t w = codes[j >> 2];
    const float a0 = (float)(int8_t)(w >> (8 * (j & 3))) * scale(j);
    const float a1 = (float)(int8_t)(w >> (8 * ((j + 1) & 3))) * scale(j + 1);
    out[j >> 1] = pack_bf16x2(a0, a1);
  }
  return out;
}

// NPRE: key tiles in flight per workgroup (register sets of the cooperative load), so a tile's global loads are
// issued NPRE tiles before its LDS store.
// NC: column tiles per workgroup; CW: column tiles per wave; KH: key halves (KH = 2: the workgroup takes two
// consecutive key chunks, each with its own NC / CW waves, and combines them before the split epilogue). The
// workgroup has KH NC / CW waves.
template <int D, int NPRE, int MODE, int KT, int CW, int NC, int KH>
__global__ void __launch_bounds__(64 * NC / CW * KH) prefill_mfma_bf16(const PrefillArgs a) {
  static_assert(KT == 32 || KT == 64, "key tiles of 32 or 64 keys");
  static_assert(CW == 1 || CW == 2, "one or two column tiles per wave");
  static_assert(NC == 8 || NC == 16, "8 or 16 column tiles per workgroup");
  static_assert(KH == 1 || (KH == 2 && CW == 1 && NC == 8), "key halves: 8 column tiles of one per wave");
  constexpr int CWV = NC / CW;                // waves of one key half
  constexpr int PW = CWV * KH, PT = 64 * PW;  // waves and threads of the workgroup
  constexpr int PTH = PT / KH;                // threads of one key half (its tiles' cooperative load)
  constexpr int MT = KT / 16, HT = KT / 32;   // 16-key row tiles, 32-key halves
  constexpr int kSlots = NC * 16;             // (column, token) rows of a split state
  constexpr int KS = D / 32, DT = D / 16, P = PrefillSmem<D>::kPitch, TE = HT * PrefillSmem<D>::kTile;
  constexpr int CH = MODE == 0 ? 8 : 16;   // channels per cooperative-load chunk: 16 bytes of bf16 or of codes
  constexpr int CPK = D / CH;               // chunks per key row
  constexpr int NCH = KT * CPK;                // chunks per K (or V) tile
  constexpr int LPT = (NCH + PTH - 1) / PTH;   // chunks per thread per K (or V) tile
  static_assert(NCH % PTH == 0 || (LPT == 1 && NCH % 64 == 0), "tile chunks must divide over whole waves");
  // the key half whose tiles this thread loads, and its index there; threads past the tile's chunks (NCH < PTH:
  // whole waves) take no part in the cooperative load
  const int hx = KH == 1 ? 0 : (int)threadIdx.x / PTH, tx = (int)threadIdx.x % PTH;
  const bool loads = NCH >= PTH || tx < NCH;
  __shared__ __align__(16) uint16_t sm[2][KH][2][TE];  // [buffer][key half][K, V][32 keys][P]
  __shared__ int bids[kMaxSplitBlocks];
  __shared__ int last_flag;

  // Units by XCD: the dispatcher deals workgroups round-robin to the 8 XCDs (workgroup L on XCD L mod 8), and
  // unit u's splits take workgroups L = u mod 8 + 8 (nsplit (u / 8) + split), so they share one L2, which then
  // serves the merge its partials. Each workgroup checks its XCD (XCC_ID); a unit any of whose splits ran
  // elsewhere is merged through memory instead. Units go out last query tile first, over all (sequence, KV
  // head) pairs: under the causal mask a unit's keys grow with its tile index, so the longest units start first.
  const int L = blockIdx.x;
  const int sp = (L >> 3) % a.nsplit;
  const int u = (L & 7) + 8 * ((L >> 3) / a.nsplit);
  if (u >= a.npair * a.qtiles) return;  // the grid is padded to whole groups of 8 units
  const int pair = u % a.npair;
  const int j = a.qtiles - 1 - u / a.npair;
  const int s = pair % a.S, h = pair / a.S;
  const int G = a.G, TT = a.tt, NT = 16 * a.tt;  // query heads, token subtiles, tokens per unit
  const int n = a.qlen[s];
  if (NT * j >= n) return;
  const int row0 = a.qstart[s] + NT * j;
  const int ctx = min(a.ctx[s], a.max_ctx);
  const int ntok = min(min(NT, n - NT * j), a.T - row0);  // rows past T are not touched
  if (ntok <= 0 || row0 < 0) return;
  const int P0 = ctx - n + NT * j;  // position of the unit's first token
  // keys [0, kv_vis) are visible to some token of the unit; this split takes [k_lo, kv_end), KH chunks of
  // a.chunk keys, key half x the x-th of them (the last half may be shorter or empty)
  const int kv_vis = max(1, min(ctx, P0 + ntok));
  const int nvalid = (kv_vis + KH * a.chunk - 1) / (KH * a.chunk);
  const int k_lo = sp * KH * a.chunk;
  if (k_lo >= kv_vis) return;
  const int kv_end = min(k_lo + KH * a.chunk, kv_vis);
  auto half_lo = [&](int x) { return min(k_lo + x * a.chunk, kv_end); };
  auto half_end = [&](int x) { return min(k_lo + (x + 1) * a.chunk, kv_end); };
  const int nblk = min((kv_end - k_lo + 15) >> 4, kMaxSplitBlocks);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wcol = wave % CWV, whalf = wave / CWV;  // the wave's column-tile slot and key half
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;

  // bf16 pools stage each block's offset in 16-byte units (the host checks that it fits 32 bits), so that a
  // tile load's address is one shift-add; INT8 pools stage block ids (their scales have strides of their own).
  const int32_t* btr = a.bt + (int64_t)s * a.bt_ss + (k_lo >> 4);
  const int last_col = a.bt_w - 1 - (k_lo >> 4);  // >= nblk - 1 when the host's width check held
  for (int i = threadIdx.x; i < nblk; i += PT) {
    const int blk = min(max(btr[min(i, last_col)], 0), a.nb - 1);
    bids[i] = MODE == 0 ? (int)(uint32_t)((uint64_t)blk * (uint64_t)(a.kv_sn >> 3)) : blk;
  }

  // Column tiles c = wcol + (NC / CW) ci of the unit: query head g = c % G of the group, tokens 16 tt .. 16 tt + 15
  // with tt = c / G (G * TT <= NC). A column tile's B operand holds token r of head g (zero past the unit's
  // tokens).
  int cg[CW], ctok[CW];
  bool cvalid[CW];  // wave-uniform
  bf16x8 qop[CW][KS];
#pragma unroll
  for (int ci = 0; ci < CW; ++ci) {
    const int c = wcol + CWV * ci;
    cg[ci] = c % G;
    ctok[ci] = 16 * (c / G);
    cvalid[ci] = c / G < TT && ctok[ci] < ntok;
    const bool valid = cvalid[ci] && ctok[ci] + r < ntok;
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)(row0 + min(ctok[ci] + r, ntok - 1)) * a.q_st +
                           (int64_t)(h * G + cg[ci]) * a.q_sh;
#pragma unroll
    for (int jj = 0; jj < KS; ++jj) {
      u32x4 qv = *(const u32x4*)(qrow + 32 * jj + 8 * q4);
      if (!valid) qv = u32x4{0, 0, 0, 0};
      qop[ci][jj] = __builtin_bit_cast(bf16x8, qv);
    }
  }
  // l_run: each column's softmax denominators as an MFMA accumulator (every row holds the column sum)
  float m_run[CW];
  f32x4 l_run[CW];
  f32x4 acc[CW][DT];
#pragma unroll
  for (int ci = 0; ci < CW; ++ci) {
    m_run[ci] = kNegInf;
    l_run[ci] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[ci][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();  // block ids staged

  // every wave runs the longest half's tile count (half 0's) for the barriers; each computes its own half's
  const int ntiles = (half_end(0) - k_lo + KT - 1) / KT;
  const int h_lo = half_lo(whalf), h_end = half_end(whalf);
  const int my_tiles = (h_end - h_lo + KT - 1) / KT;
  // Cooperative tile load: chunk c = threadIdx.x + 256 i of the KT x D tile is key c / CPK, channels
  // CH (c % CPK) ..; keys past kv_end re-read the split's last key (finite values that the mask zeroes). Plain
  // (temporal) loads: every query tile of the sequence reads the same keys, so L2 keeps serving them.
  // INT8 pools: the chunk's 8 codes of K and of V with their scales; the LDS store dequantizes them to bf16,
  // q * s in fp32 rounded to bf16, the values the reference's gather path attends over. Format B's keys at or
  // past the sequence's last full block come from its bf16 staging slot instead.
  const int nq = MODE == 2 ? ctx / 16 * 16 : 0;
  const int tail = MODE == 2 ? min(a.tails[s], a.n_stage - 1) : -1;
  KvRaw<MODE> raw[NPRE][LPT];
  const uint16_t* kbase = (const uint16_t*)a.k + (int64_t)h * a.kv_sh;  // MODE 0: the KV head's planes
  const uint16_t* vbase = (const uint16_t*)a.v + (int64_t)h * a.kv_sh;
  // keys past the half's end (an empty half: past the split's) re-read its last key
  const int rel_lo = half_lo(hx) - k_lo, rel_cap = max(half_end(hx), half_lo(hx) + 1) - 1 - k_lo;
  auto gload = [&](int set, int t) {
    if (!loads) return;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tx + PTH * i, cg = c % CPK;
      const int rel = min(rel_lo + KT * t + c / CPK, min(rel_cap, kv_end - 1 - k_lo));  // key offset in the split
      const int off = rel & 15;
      KvRaw<MODE>& x = raw[set][i];
      if constexpr (MODE == 0) {
        const int64_t e = (int64_t)(uint32_t)bids[rel >> 4] * 8 + (off * D + 8 * cg);
        x.k = *(const u32x4*)(kbase + e);
        x.v = *(const u32x4*)(vbase + e);
      } else {
        const int64_t blk = bids[rel >> 4];
        const int64_t e = (int64_t)h * a.kv_sh + blk * a.kv_sn + off * D + CH * cg;
        x.k = *(const u32x4*)((const int8_t*)a.k + e);
        x.v = *(const u32x4*)((const int8_t*)a.v + e);
        x.vs = scale_bits(a.vs, a.vs_f32, (int64_t)h * a.vs_sh + blk * a.vs_sn + off);
        if constexpr (MODE == 1) {
          x.ks = scale_bits(a.ks, a.ks_f32, (int64_t)h * a.ks_sh + blk * a.ks_sn + off);
        } else {
          const int64_t sb = (int64_t)h * a.ks_sh + blk * a.ks_sn + CH * cg;  // the chunk's 16 channel scales
          if (a.ks_vec) {  // 16-byte aligned rows (host-checked): 32 or 64 contiguous bytes
            const u32x4* src = (const u32x4*)((const uint8_t*)a.ks + sb * (a.ks_f32 ? 4 : 2));
            x.ks[0] = src[0];
            x.ks[1] = src[1];
            if (a.ks_f32) {
              x.ks[2] = src[2];
              x.ks[3] = src[3];
            }
          } else {
#pragma unroll
            for (int j = 0; j < 16; j += 2) {
              const uint32_t b0 = scale_bits(a.ks, a.ks_f32, sb + j), b1 = scale_bits(a.ks, a.ks_f32, sb + j + 1);
              if (a.ks_f32) {
                x.ks[j >> 2][j & 3] = b0;
                x.ks[j >> 2][(j & 3) + 1] = b1;
              } else {
                x.ks[j >> 3][(j >> 1) & 3] = b0 | (b1 << 16);
              }
            }
          }
          const int pos = k_lo + rel;
          x.staged = tail >= 0 && pos >= nq;
          if (x.staged) {
            const u32x4* st = (const u32x4*)(a.stage + (int64_t)h * a.st_sh + (int64_t)tail * a.st_sn +
                                             (int64_t)(pos & 15) * a.st_sb + CH * cg);
            x.st[0] = st[0];
            x.st[1] = st[1];
          }
        }
      }
    }
  };
  auto sstore = [&](int set, int buf) {
    if (!loads) return;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tx + PTH * i;
      const int e = (c / CPK) * P + CH * (c % CPK);
      const KvRaw<MODE>& x = raw[set][i];
      if constexpr (MODE == 0) {
        *(u32x4*)(&sm[buf][hx][0][e]) = x.k;
        *(u32x4*)(&sm[buf][hx][1][e]) = x.v;
      } else {
        const u32x2 klo = {x.k[0], x.k[1]}, khi = {x.k[2], x.k[3]};
        const u32x2 vlo = {x.v[0], x.v[1]}, vhi = {x.v[2], x.v[3]};
        const float vsf = scale_value(x.vs, a.vs_f32);
        *(u32x4*)(&sm[buf][hx][1][e]) = dequant8(vlo, [&](int) { return vsf; });
        *(u32x4*)(&sm[buf][hx][1][e + 8]) = dequant8(vhi, [&](int) { return vsf; });
        if constexpr (MODE == 1) {
          const float ksf = scale_value(x.ks, a.ks_f32);
          *(u32x4*)(&sm[buf][hx][0][e]) = dequant8(klo, [&](int) { return ksf; });
          *(u32x4*)(&sm[buf][hx][0][e + 8]) = dequant8(khi, [&](int) { return ksf; });
        } else {
          *(u32x4*)(&sm[buf][hx][0][e]) =
              x.staged ? x.st[0] : dequant8(klo, [&](int j) { return chan_scale(x.ks, a.ks_f32, j); });
          *(u32x4*)(&sm[buf][hx][0][e + 8]) =
              x.staged ? x.st[1] : dequant8(khi, [&](int j) { return chan_scale(x.ks, a.ks_f32, 8 + j); });
        }
      }
    }
  };
  const int tr_off = tr16_offset(r, q4, P);
  const bf16x8 kOnes = {(__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f,
                        (__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f};
  constexpr float kRescaleSlack = 8.f;  // p <= 2^8 against the lazily raised max (as in the decode kernel)
  // p <= 2^16 against a max left as it stands: O stays finite for |v| < 2^94 over 2^17 keys
  constexpr float kFastRange = 16.f;
  const float inv_scale_log2 = 1.f / a.scale_log2;
  float fast_thr[CW], m_off[CW];  // m_off: the exponentials' offset, m_run or 0 while m_run is -inf
#pragma unroll
  for (int ci = 0; ci < CW; ++ci) fast_thr[ci] = kNegInf, m_off[ci] = 0.f;
  // The all-ones operand of the row sums, opaque to the compiler so that it stays in registers instead of being
  // rematerialized for every tile.
  bf16x8 ones = kOnes;
  asm volatile("" : "+v"(ones));

  auto tile = [&](int t) {
    const int buf = t & 1;
    const int t0 = h_lo + KT * t;
    const bool masked = t0 + KT - 1 > P0 || t0 + KT > h_end;  // some key of the tile is hidden from some token
    const uint16_t* ks = sm[buf][whalf][0];
    const uint16_t* vs = sm[buf][whalf][1];
    // The K operands of the tile serve both column tiles of the wave.
    bf16x8 kop[MT][KS];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int jj = 0; jj < KS; ++jj) kop[mt][jj] = *(const bf16x8*)(ks + (16 * mt + r) * P + 32 * jj + 8 * q4);
    // An unused column tile (G < 8) skips its scores and softmax (the VALU work, which bounds the kernel when
    // three workgroups share a CU) and takes zero probabilities, so that the P.V MFMAs below run for every
    // column without a branch between them and the V reads run ahead of them (per-column branches there cost
    // 2.2 us of a 512-token chunk at 8K context).
    bf16x8 pop[CW][HT];
#pragma unroll
    for (int ci = 0; ci < CW; ++ci) {
      if (!cvalid[ci]) {  // wave-uniform
#pragma unroll
        for (int hf = 0; hf < HT; ++hf) pop[ci][hf] = bf16x8{};
        continue;
      }
      f32x4 sc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        sc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < KS; ++jj)
          sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[mt][jj], qop[ci][jj], sc[mt], 0, 0, 0);
      }
      if (masked) {
        // row (mt, q4, i) holds key t0 + 16 mt + 4 q4 + i: hidden past the token's position or the half's end
        const int lim = min(P0 + ctok[ci] + r, h_end - 1) - t0 - 4 * q4;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * mt + i > lim) sc[mt][i] = kNegInf;
      }
      // Each lane's largest score (the tile's max needs two cross-lane steps more).
      float lmax;
      if constexpr (MT == 4) {  // 16 scores in 8 three-input maxima
        auto m3 = [](float x, float y, float z) { return vmax(vmax(x, y), z); };
        const float a0 = m3(sc[0][0], sc[0][1], sc[0][2]), a1 = m3(sc[0][3], sc[1][0], sc[1][1]);
        const float a2 = m3(sc[1][2], sc[1][3], sc[2][0]), a3 = m3(sc[2][1], sc[2][2], sc[2][3]);
        const float a4 = m3(sc[3][0], sc[3][1], sc[3][2]);
        lmax = vmax(m3(a0, a1, sc[3][3]), m3(a2, a3, a4));
      } else {
        lmax = kNegInf;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          lmax = vmax(lmax, vmax(vmax(sc[mt][0], sc[mt][1]), vmax(sc[mt][2], sc[mt][3])));
      }
      // The tile's max is taken only when some score exceeds the running max by more than kFastRange (fast_thr,
      // in raw score units; -inf while a token has no max yet, so a wave's first visible scores always take it):
      // otherwise every p is at most 2^kFastRange against the running max as it stands, and the exponentials use
      // it unchanged (the lazily raised max would mostly leave it too). Two cross-lane swaps, a multiply and a
      // compare per tile fewer: 512 new tokens at 8K context 28.2 -> 27.2 us, four 2048-token prompts 48.1 ->
      // 46.1, the same over INT8 pools 32.7 -> 31.1.
      if (__builtin_amdgcn_ballot_w64(lmax > fast_thr[ci])) {
        const float mx = max_over_rows_swap(lmax) * a.scale_log2;
        // A token of a later split may see none of the keys so far (m_run = -inf, l = 0, acc = 0): the offsets
        // below are taken as 0 then, so that -inf - -inf never forms.
        if (__builtin_amdgcn_ballot_w64(mx > m_run[ci] + kRescaleSlack)) {
          const float m_new = fmaxf(m_run[ci], mx);
          const float alpha = fast_exp2(m_run[ci] - (m_new == kNegInf ? 0.f : m_new));  // 0 while m_run is -inf
          l_run[ci] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[ci][dt] *= alpha;
          m_run[ci] = m_new;
          m_off[ci] = m_new == kNegInf ? 0.f : m_new;
          fast_thr[ci] = (m_new + kFastRange) * inv_scale_log2;
        }
      }
#pragma unroll
      for (int hf = 0; hf < HT; ++hf)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          pop[ci][hf][i] = (__bf16)fast_exp2(fmaf(sc[2 * hf + (i >> 2)][i & 3], a.scale_log2, -m_off[ci]));
      // The denominators on the matrix cores: ones . P^T sums each token's bf16 probabilities (the values the
      // P.V product uses) into every row of l_run, in place of VALU adds and a cross-row reduction.
#pragma unroll
      for (int hf = 0; hf < HT; ++hf)
        l_run[ci] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pop[ci][hf], l_run[ci], 0, 0, 0);
    }
    // V^T operands (32 keys each), each shared by both column tiles.
#pragma unroll
    for (int hf = 0; hf < HT; ++hf)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 vop = read_v_operand<bf16x8>(vs + 32 * P * hf, tr_off, P, 16 * dt);
#pragma unroll
        for (int ci = 0; ci < CW; ++ci)
          acc[ci][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[ci][hf], acc[ci][dt], 0, 0, 0);
      }
  };

  // Register set k % NPRE carries tile k from its global loads to its LDS store; LDS is double-buffered (tile t
  // in buffer t & 1). The set of tile t is free once tile t is in LDS, and is refilled with tile t + NPRE. The
  // loads are issued unconditionally (past the last tile they re-read the split's last key), so that the wait
  // before each LDS store is a fixed count that leaves the NPRE - 1 younger sets in flight.
  // in ring order (the compiler would otherwise issue set 0's V after set 1, and the first store would wait for
  // both sets)
#pragma unroll
  for (int k = 0; k < NPRE; ++k) {
    gload(k, k);
    asm volatile("" ::: "memory");
  }
  sstore(0, 0);
  __syncthreads();
  // Whole passes of NPRE tiles, then the last ntiles % NPRE tiles outside the loop: an exit from the middle of a
  // pass would reach the loop head (in the compiler's control flow) with a register set's loads outstanding, and
  // every pass would then wait for its next tile's loads before issuing the ones after it.
  int tb = 0;
  for (; tb + NPRE <= ntiles; tb += NPRE) {
#pragma unroll
    for (int k = 0; k < NPRE; ++k) {
      const int t = tb + k;
      gload(k, t + NPRE);
      if (KH == 1 || t < my_tiles) tile(t);  // wave-uniform
      // buffer (t + 1) & 1 was last read in tile t - 1, before the last barrier (after the last tile: the
      // re-read last key, never used)
      sstore((k + 1) % NPRE, (t + 1) & 1);
      __syncthreads();
    }
  }
  // their loads, and the first one's LDS store, were issued in the loop
#pragma unroll
  for (int k = 0; k < NPRE - 1; ++k) {
    const int t = tb + k;
    if (t >= ntiles) break;
    if (KH == 1 || t < my_tiles) tile(t);
    if (t + 1 < ntiles) sstore((k + 1) % NPRE, (t + 1) & 1);
    __syncthreads();
  }

  float lsum[CW];  // token r's denominators (every row of the l_run accumulator holds the same sum)
#pragma unroll
  for (int ci = 0; ci < CW; ++ci) lsum[ci] = l_run[ci][0];
  if constexpr (KH == 2) {
    // Key half 1's waves hand their state to half 0's waves of the same column tile through LDS (the tile
    // buffers, free after the loop's last barrier), which combine the two like two splits: M = max(m0, m1),
    // x = 2^(m0 - M) x0 + 2^(m1 - M) x1 for l and O. A half that saw no key of a token has (-inf, 0, 0).
    constexpr int XS = DT * 4 + 2;  // floats per lane: O, m, l
    static_assert(CWV * 64 * XS * 4 <= (int)sizeof(sm), "half state fits the tile buffers");
    float* xs = (float*)&sm[0][0][0][0] + (wcol * 64 + lane) * XS;
    if (whalf == 1 && cvalid[0]) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *(f32x4*)(xs + 4 * dt) = acc[0][dt];
      xs[4 * DT] = m_run[0];
      xs[4 * DT + 1] = lsum[0];
    }
    __syncthreads();
    if (whalf == 0 && cvalid[0]) {
      const float m1 = xs[4 * DT], l1 = xs[4 * DT + 1];
      const float M = fmaxf(m_run[0], m1);
      if (M != kNegInf) {
        const float f0 = fast_exp2(m_run[0] - M), f1 = fast_exp2(m1 - M);  // 0 for a keyless half
        lsum[0] = f0 * lsum[0] + f1 * l1;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[0][dt] = f0 * acc[0][dt] + f1 * *(const f32x4*)(xs + 4 * dt);
        m_run[0] = M;
      }
    }
  }
  // the column tiles' state is half 0's now: half 1's waves only take part in the barriers and the merge
  const bool owner = KH == 1 || whalf == 0;
  if (nvalid > 1) {
    // This split's state for column c, token r: m, l at slot 16 c + r, and the split's own output O / l (the
    // weighted mean of its V rows, so fp16 holds it to 2^-11 relative) at channels 16 dt + 4 q4 .. of that row:
    // half the bytes of unnormalised fp32 partials, which the merge reads back in one or two memory round trips.
    // A row whose largest |O / l| reaches 2^15 (V values beyond fp16's range) is stored times 2^-e, so that it
    // stays below 65504, with e in l's low mantissa bits; the merge scales the row back exactly.
    const int64_t base = ((int64_t)u * a.nsplit + sp) * kSlots;
    const int split_bytes = kSlots * D * 2;
    const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
        (uint16_t*)a.part + (int64_t)u * a.nsplit * kSlots * D, (short)0, a.nsplit * split_bytes, 0x00020000);
#pragma unroll
    for (int ci = 0; ci < CW; ++ci) {
      if (!owner || !cvalid[ci] || ctok[ci] + r >= ntok) continue;
      const int slot = 16 * (wcol + CWV * ci) + r;
      const float inv = lsum[ci] > 0.f ? 1.f / lsum[ci] : 0.f;  // l = 0: the token sees no key of this split
      // the row's largest |O / l|: this lane's 4 DT channels, then the row's other three lanes (q4)
      float big = 0.f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        big = vmax(big, vmax(vmax(fabsf(acc[ci][dt][0]), fabsf(acc[ci][dt][1])),
                             vmax(fabsf(acc[ci][dt][2]), fabsf(acc[ci][dt][3]))));
      big = max_over_rows_swap(big * inv);
      // big < 2^ex; e = ex - 15 keeps the row under 2^15 (inf and NaN rows keep e = 0 and stay inf and NaN)
      const int e = big < 32768.f ? 0 : max(__builtin_amdgcn_frexp_expf(big) - 15, 0);
      const float inv_e = __builtin_amdgcn_ldexpf(inv, -e);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4 o = acc[ci][dt] * inv_e;
        const u32x2 h = {pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
        __builtin_amdgcn_raw_buffer_store_b64(h, rows, sp * split_bytes + (slot * D + 16 * dt + 4 * q4) * 2, 0,
                                              kAuxSc1);
      }
      if (q4 == 0) {
        // e (at most 113) in the low 8 bits of l's mantissa: l changes by less than 2^-15 relative
        store_coherent(a.pm + base + slot, m_run[ci]);
        store_coherent(a.pl + base + slot, __uint_as_float((__float_as_uint(lsum[ci]) & ~0xffu) | (uint32_t)e));
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      // Arrival: +1, and +2^16 from a workgroup that is not on its unit's XCD. The last to arrive merges from
      // its L2 (L1 bypassed) when every split of the unit, itself included, ran on that XCD: their write-through
      // stores updated that L2. Otherwise from memory, as agent-coherent loads.
      uint32_t xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      const int away = a.mem_merge || (int)(xcc & 0xf) != (L & 7);
      const int prev = __hip_atomic_fetch_add(a.counters + u, 1 + (away << 16), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      last_flag = (prev & 0xffff) == nvalid - 1 ? 1 + ((prev >> 16) + away == 0) : 0;
    }
    __syncthreads();
    if (!last_flag) return;
    const bool from_l2 = last_flag == 2;
    // The last split to arrive merges every split's state: thread t takes row t / TPR (column c, token rr) and
    // 1 / TPR of its channels, in batches of up to 32 channels; per round of KB splits it reads the row's m and l and
    // keeps all of the round's channel loads in flight together. KB and the batch width hold the merge's
    // registers under what the key loop needs, so the merge costs no occupancy. AUX: the loads' cache policy.
    const __amdgpu_buffer_rsrc_t mrows = __builtin_amdgcn_make_buffer_rsrc(
        a.pm + (int64_t)u * a.nsplit * kSlots, (short)0, a.nsplit * kSlots * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t lrows = __builtin_amdgcn_make_buffer_rsrc(
        a.pl + (int64_t)u * a.nsplit * kSlots, (short)0, a.nsplit * kSlots * 4, 0x00020000);
    auto merge = [&](auto aux_tag) {
      constexpr int AUX = decltype(aux_tag)::value;
      constexpr int TPR = PT / kSlots, CPT = D / TPR, CB = CPT < 32 ? CPT : 32, KB = 4;  // threads per row
      const int slot = threadIdx.x / TPR, part = threadIdx.x % TPR;
      const int c = slot >> 4, rr = slot & 15;
      const int g = c % G, tok = 16 * (c / G) + rr;
      if (c / G < TT && tok < ntok) {
        uint16_t* orow = (uint16_t*)a.out + (int64_t)(row0 + tok) * a.o_st + (int64_t)(h * G + g) * a.o_sh;
        for (int c0 = CPT * part; c0 < CPT * (part + 1); c0 += CB) {
          float M = kNegInf, den = 0.f;
          f32x4 num[CB / 4];
#pragma unroll
          for (int qd = 0; qd < CB / 4; ++qd) num[qd] = f32x4{0.f, 0.f, 0.f, 0.f};
          for (int j0 = 0; j0 < nvalid; j0 += KB) {
            float mj[KB], lj[KB];
            int ej[KB];  // their rows were stored times 2^-e
            u32x2 oj[KB][CB / 4];
#pragma unroll
            for (int uu = 0; uu < KB; ++uu) {
              const int j = min(j0 + uu, nvalid - 1);  // entries past nvalid re-read the last split, weight 0
              mj[uu] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                     mrows, (j * kSlots + slot) * 4, 0, AUX));
              const uint32_t lb = __builtin_amdgcn_raw_buffer_load_b32(lrows, (j * kSlots + slot) * 4, 0, AUX);
              lj[uu] = __uint_as_float(lb & ~0xffu);
              ej[uu] = (int)(lb & 0xffu);
#pragma unroll
              for (int qd = 0; qd < CB / 4; ++qd)
                oj[uu][qd] = __builtin_amdgcn_raw_buffer_load_b64(
                    rows, j * split_bytes + (slot * D + c0 + 4 * qd) * 2, 0, AUX);
            }
#pragma unroll
            for (int uu = 0; uu < KB; ++uu)
              if (j0 + uu >= nvalid) mj[uu] = kNegInf;
            float mb = M;
#pragma unroll
            for (int uu = 0; uu < KB; ++uu) mb = fmaxf(mb, mj[uu]);
            const float rescale = fast_exp2(M - mb);  // 0 on the first round (split 0 holds the row's first key)
            den *= rescale;
#pragma unroll
            for (int qd = 0; qd < CB / 4; ++qd) num[qd] *= rescale;
#pragma unroll
            for (int uu = 0; uu < KB; ++uu) {
              const float w = fast_exp2(mj[uu] - mb) * lj[uu];  // 0 for padding entries and keyless splits
              den += w;
              const float wo = __builtin_amdgcn_ldexpf(w, ej[uu]);
#pragma unroll
              for (int qd = 0; qd < CB / 4; ++qd) {
                const u32x2 hw = oj[uu][qd];
                const f32x4 o = {f16_bits_to_f32(hw[0] & 0xffffu), f16_bits_to_f32(hw[0] >> 16),
                                 f16_bits_to_f32(hw[1] & 0xffffu), f16_bits_to_f32(hw[1] >> 16)};
                num[qd] += wo * o;
              }
            }
            M = mb;
          }
          const float inv = 1.f / den;
#pragma unroll
          for (int qd = 0; qd < CB / 4; qd += 2) {
            const f32x4 x = num[qd] * inv, y = num[qd + 1] * inv;
            *(u32x4*)(orow + c0 + 4 * qd) =
                u32x4{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(y[0], y[1]),
                      pack_bf16x2(y[2], y[3])};
          }
        }
      }
    };
    if (from_l2) {
      asm volatile("buffer_inv sc0" ::: "memory");  // sc0 loads may hit the CU's L1: drop any earlier copy first
      merge(std::integral_constant<int, kAuxSc0>());
    } else
      merge(std::integral_constant<int, kAuxSc1>());
    if (threadIdx.x == 0)
      __hip_atomic_store(a.counters + u, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // One split: token r's output for each column tile is acc / l.
#pragma unroll
  for (int ci = 0; ci < CW; ++ci) {
    if (!owner || !cvalid[ci] || ctok[ci] + r >= ntok) continue;
    const float inv = 1.f / lsum[ci];
    uint16_t* orow = (uint16_t*)a.out + (int64_t)(row0 + ctok[ci] + r) * a.o_st + (int64_t)(h * G + cg[ci]) * a.o_sh;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint32_t lo = pack_bf16x2(acc[ci][dt][0] * inv, acc[ci][dt][1] * inv);
      const uint32_t hi2 = pack_bf16x2(acc[ci][dt][2] * inv, acc[ci][dt][3] * inv);
      *(u32x2*)(orow + 16 * dt + 4 * q4) = u32x2{lo, hi2};
    }
  }
}

}  // namespace sipa

using namespace sipa;

static bool aligned16p(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Keys per split for a requested split count: ceil(max_context / splits) rounded up to a multiple of 64 (the key
// tile), at least 256; the launch then has ceil(max_context / chunk) splits.
static int prefill_chunk(int max_context, int splits) {
  splits = std::max(1, std::min(splits, kPrefillMaxSplits));
  const int c = (max_context + splits - 1) / splits;
  return std::max(256, (c + 63) / 64 * 64);
}

// Split count policy: about two workgroups per CU over all units (units = KV heads x query tiles of
// 16 tokens), no split under 256 keys, at most 32.
static int prefill_splits_host(int64_t units, int max_context, int cu_count) {
  if (units <= 0 || max_context <= 0) return 1;
  const int64_t target = 2LL * std::max(cu_count, 1);
  const int want = (int)std::min<int64_t>((target + units - 1) / units, kPrefillMaxSplits);
  const int chunk = prefill_chunk(max_context, want);
  return (max_context + chunk - 1) / chunk;
}

struct PrefillLayout {
  int64_t counters, pm, pl, part, total;  // byte offsets into the workspace
};

static PrefillLayout prefill_layout(int64_t units, int nsplit, int D, int nc) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  PrefillLayout l;
  const int64_t rows = units * nsplit * nc * 16;
  l.counters = 0;
  l.pm = kCounterBytes;
  l.pl = l.pm + up(rows * 4);
  l.part = l.pl + up(rows * 4);
  l.total = l.part + up(rows * D * 2);  // fp16 partial outputs
  return l;
}

extern "C" int32_t sipa_prefill_splits(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                       int64_t query_tiles, int32_t max_context, int32_t cu_count) {
  if (num_kv_heads <= 0 || num_q_heads < num_kv_heads) return 1;
  if (cu_count <= 0) cu_count = sipa_device_cu_count(-1);
  const int tt = prefill_subtiles(num_q_heads / num_kv_heads, 8);
  return prefill_splits_host((int64_t)num_kv_heads * ((query_tiles + tt - 1) / tt), max_context, cu_count);
}

extern "C" int64_t sipa_prefill_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                                                int32_t head_dim, int32_t max_query_len, int32_t max_context,
                                                int32_t num_splits) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads < num_kv_heads || max_query_len <= 0 || max_context <= 0)
    return 0;
  const int chunk = prefill_chunk(max_context, num_splits);
  const int nsplit = (max_context + chunk - 1) / chunk;
  if (nsplit <= 1) return 0;
  int64_t most = 0;  // the largest over the workgroup layouts sipa_prefill may pick
  for (const int nc : {8, 16}) {
    const int nt = 16 * prefill_subtiles(num_q_heads / num_kv_heads, nc);
    const int64_t units = (int64_t)num_seqs * num_kv_heads * ((max_query_len + nt - 1) / nt);
    most = std::max(most, prefill_layout(units, nsplit, head_dim, nc).total);
  }
  return most;
}

template <int D, int NPRE, int KT, int CW, int NC, int KH>
static void launch_prefill(int mode, dim3 grid, hipStream_t st, const PrefillArgs& a) {
  const dim3 block(64 * NC / CW * KH);
  if (mode == SIPA_KV_PLAIN)
    hipLaunchKernelGGL((prefill_mfma_bf16<D, NPRE, 0, KT, CW, NC, KH>), grid, block, 0, st, a);
  else if (mode == SIPA_KV_INT8_TOKEN)
    hipLaunchKernelGGL((prefill_mfma_bf16<D, NPRE, 1, KT, CW, NC, KH>), grid, block, 0, st, a);
  else if constexpr (NC == 8 && KH == 1)  // format B in 16-wave workgroups is refused by the host (registers)
    hipLaunchKernelGGL((prefill_mfma_bf16<D, NPRE, 2, KT, CW, NC, KH>), grid, block, 0, st, a);
}

extern "C" int32_t sipa_prefill(const sipa_prefill_params* p, void* stream) {
  SIPA_CHECK(p != nullptr && p->struct_size == (int32_t)sizeof(sipa_prefill_params), SIPA_EINVAL,
             "struct_size does not match this library's sipa_prefill_params (%d bytes)",
             (int)sizeof(sipa_prefill_params));
  const int S = p->num_seqs, Hq = p->num_q_heads, Hkv = p->num_kv_heads, D = p->head_dim;
  if (S == 0 || p->max_query_len == 0) return SIPA_OK;
  SIPA_CHECK(S > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, SIPA_EINVAL, "bad sequence or head counts");
  const int G = Hq / Hkv;
  SIPA_CHECK(G <= kPrefillMaxGroup, SIPA_EUNSUPPORTED, "GQA group %d > %d", G, kPrefillMaxGroup);
  SIPA_CHECK(D == 64 || D == 128, SIPA_EUNSUPPORTED, "head_dim %d not in {64, 128}", D);
  SIPA_CHECK(p->scale > 0.f && p->scale < __builtin_inff(), SIPA_EINVAL,
             "scale %g must be positive and finite (the kernel takes maxima of the unscaled scores)", (double)p->scale);
  SIPA_CHECK(p->block_size == 16, SIPA_EUNSUPPORTED, "block_size %d != 16", p->block_size);
  SIPA_CHECK(p->max_context > 0 && p->max_context <= kMaxSplitBlocks * 16, SIPA_EUNSUPPORTED,
             "max_context %d outside [1, %d]", p->max_context, kMaxSplitBlocks * 16);
  SIPA_CHECK(p->max_query_len > 0, SIPA_EINVAL, "max_query_len %d", p->max_query_len);
  SIPA_CHECK(p->bt_width > 0 && (int64_t)p->bt_width * 16 >= p->max_context, SIPA_EINVAL,
             "block_tables rows of %d entries cannot cover max_context %d", p->bt_width, p->max_context);
  SIPA_CHECK(p->q && p->k_cache && p->v_cache && p->block_tables && p->context_lens && p->query_starts &&
                 p->query_lens && p->out, SIPA_EINVAL, "NULL pointer");
  SIPA_CHECK(aligned16p(p->q) && p->q_stride_t % 8 == 0 && p->q_stride_h % 8 == 0, SIPA_EINVAL,
             "q rows must be 16-byte aligned");
  SIPA_CHECK(aligned16p(p->out) && p->out_stride_t % 8 == 0 && p->out_stride_h % 8 == 0, SIPA_EINVAL,
             "out rows must be 16-byte aligned");
  SIPA_CHECK(p->num_tokens > 0 && p->num_blocks > 0, SIPA_EINVAL, "num_tokens %d, num_blocks %d",
             p->num_tokens, p->num_blocks);
  const int mode = p->kv_mode;
  SIPA_CHECK(mode == SIPA_KV_PLAIN || mode == SIPA_KV_INT8_TOKEN || mode == SIPA_KV_INT8_KCHAN, SIPA_EINVAL,
             "kv_mode %d", mode);
  SIPA_CHECK(aligned16p(p->k_cache) && aligned16p(p->v_cache) && p->kv_stride_h % 8 == 0 &&
                 p->kv_stride_n % 8 == 0, SIPA_EINVAL, "K/V pools must be 16-byte aligned");
  SIPA_CHECK(mode != SIPA_KV_PLAIN || (int64_t)(p->num_blocks - 1) * (p->kv_stride_n / 8) <= 0xffffffffLL,
             SIPA_EUNSUPPORTED, "bf16 pool blocks must lie within 64 GiB of the head's first block (%d blocks of "
             "stride %lld)", p->num_blocks, (long long)p->kv_stride_n);
  if (mode != SIPA_KV_PLAIN) {
    SIPA_CHECK(p->k_scale && p->v_scale, SIPA_EINVAL, "INT8 pools need k_scale and v_scale");
    SIPA_CHECK((p->k_scale_dtype == SIPA_F16 || p->k_scale_dtype == SIPA_F32) &&
                   (p->v_scale_dtype == SIPA_F16 || p->v_scale_dtype == SIPA_F32),
               SIPA_EUNSUPPORTED, "scales must be fp16 or fp32");
    const int ksz = p->k_scale_dtype == SIPA_F32 ? 4 : 2, vsz = p->v_scale_dtype == SIPA_F32 ? 4 : 2;
    SIPA_CHECK(((uintptr_t)p->k_scale % ksz) == 0 && ((uintptr_t)p->v_scale % vsz) == 0, SIPA_EINVAL,
               "scales must be aligned to their element size");
    if (mode == SIPA_KV_INT8_KCHAN)
      SIPA_CHECK(p->stage && p->tail_slots && p->num_stage > 0 && aligned16p(p->stage) && p->st_stride_h % 8 == 0 &&
                     p->st_stride_n % 8 == 0 && p->st_stride_b % 8 == 0,
                 SIPA_EINVAL, "format B needs a 16-byte aligned bf16 staging pool and tail slots");
  }
  SIPA_CHECK(p->wg_layout >= SIPA_PREFILL_AUTO && p->wg_layout <= SIPA_PREFILL_W16H2, SIPA_EINVAL,
             "wg_layout %d is not a SIPA_PREFILL_* layout", p->wg_layout);
  // The split count and the layout choice are made over 8-column units; a 16-column layout then runs half as
  // many units with the same splits.
  const int tt8 = prefill_subtiles(G, 8);
  const int64_t units8 = (int64_t)S * Hkv * ((p->max_query_len + 16 * tt8 - 1) / (16 * tt8));
  const int cus = sipa_device_cu_count(-1);
  int splits = p->num_splits;
  if (splits <= 0) splits = prefill_splits_host(units8, p->max_context, cus);
  const int chunk = prefill_chunk(p->max_context, splits);
  const int nchunk = (p->max_context + chunk - 1) / chunk;  // key chunks per unit
  // split launches: whole groups of 8 units, one XCD each (the kernel's workgroup-to-unit mapping); a
  // workgroup of KH key halves takes KH consecutive chunks
  auto grid_of = [&](int64_t units, int kh) {
    const int ns = (nchunk + kh - 1) / kh;
    return (ns > 1 ? (units + 7) / 8 * 8 : units) * ns;
  };
  // Layout (SIPA_PREFILL_AUTO), from g8, the grid of 8-column workgroups (warm A/B on one MI355X, 0.5B and 1.5B
  // shapes, us per call):
  //  - g8 <= CUs: 8-wave workgroups, one per CU (16-wave ones would leave half the CUs idle).
  //  - a chunk at least its own length into its context (balanced units: the causal triangle varies a unit's keys
  //    by at most a factor of two):
  //    . bf16 pools, 8 or more key chunks of at most 1024 keys: 16 waves over 8 column tiles and two consecutive
  //      key chunks (INT8 pools: each half dequantizes its own tiles, twice the store work per CU; 512 at 8K
  //      32.4 -> 34.8, so they keep W16X1),
  //      combined in the workgroup, so that half as many splits store partials and merge (one merging workgroup
  //      per unit reads 4 partials, not 8): 512 new tokens at 8K 29.0 -> 28.2, 256 at 8K 23.1 -> 20.5, 128 at 8K
  //      25.5 -> 18.5, at head_dim 128 512 at 8K 46.5 -> 43.8, 256 at 8K 39.2 -> 30.1 (best of the others ->);
  //    . otherwise, with one chunk or chunks of at least 1024 keys: 16-wave workgroups of 16 column tiles, one per
  //      CU at a time. Two co-resident 8-column workgroups do not share a CU evenly (the later-dispatched ran ~30%
  //      longer and finished alone), and 16 column tiles share each K/V tile load: 512 new tokens at 16K
  //      48.9 -> 46.3 (8-wave), 16 chunks of 512 at 8K 313.8 -> 290.6 (4-wave), 1024 at 8K 47.2 -> 44.0;
  //    . else 8-wave workgroups.
  //  - fresh prompts: 8-wave workgroups up to 3 per CU (two 2048-token prompts 31.9 against 40.3 at 16 waves:
  //    32-token units double the longest CU's keys); above, 16-wave ones (four 2048-token prompts 48.6 against
  //    50.4 at 4 waves; at head_dim 128 76.0 against 87.9), except at head_dim 64 beyond 4 per CU, where 4-wave
  //    workgroups of two column tiles per wave share each K/V operand read among more tokens (six prompts 67.3
  //    against 76.9; at head_dim 128 their 206 registers leave two waves per SIMD, never the best).
  // Format B's one-column waves hold too many registers for 16 waves; it takes the 4-wave layout.
  int layout = p->wg_layout;
  if (layout == SIPA_PREFILL_AUTO) {
    const int64_t g8 = grid_of(units8, 1);
    const bool balanced = p->max_context >= 2LL * p->max_query_len;
    if (mode == SIPA_KV_INT8_KCHAN) layout = SIPA_PREFILL_W4X2;
    else if (g8 <= cus) layout = SIPA_PREFILL_W8X1;
    else if (balanced)
      layout = mode == SIPA_KV_PLAIN && nchunk >= 8 && chunk <= 1024 ? SIPA_PREFILL_W16H2
               : nchunk == 1 || chunk >= 1024                      ? SIPA_PREFILL_W16X1
                                                                   : SIPA_PREFILL_W8X1;
    else if (g8 <= 3LL * cus) layout = SIPA_PREFILL_W8X1;
    else if (D == 64 && g8 > 4LL * cus) layout = SIPA_PREFILL_W4X2;
    else layout = SIPA_PREFILL_W16X1;
  }
  SIPA_CHECK(mode != SIPA_KV_INT8_KCHAN || layout == SIPA_PREFILL_W4X2 || layout == SIPA_PREFILL_W8X1,
             SIPA_EUNSUPPORTED, "format B pools take SIPA_PREFILL_W4X2 or _W8X1 (16-wave workgroups cannot hold "
             "their registers)");
  const PfShape shape = prefill_shape(layout);
  const int tt = prefill_subtiles(G, shape.nc);
  const int qtiles = (p->max_query_len + 16 * tt - 1) / (16 * tt);
  const int64_t units = (int64_t)S * Hkv * qtiles;
  const int nsplit = (nchunk + shape.kh - 1) / shape.kh;  // workgroups per unit
  const int64_t wgs = grid_of(units, shape.kh);
  SIPA_CHECK(wgs <= 0x7fffffff, SIPA_EINVAL, "%lld workgroups exceed the grid limit", (long long)wgs);
  PrefillLayout lay{};
  if (nsplit > 1) {
    SIPA_CHECK(units <= kMaxCounters, SIPA_EINVAL,
               "%lld query tiles x KV heads exceed the %d merge counters of a split launch; use one split",
               (long long)units, kMaxCounters);
    lay = prefill_layout(units, nsplit, D, shape.nc);
    SIPA_CHECK(p->workspace != nullptr && ((uintptr_t)p->workspace & 255) == 0 && p->workspace_bytes >= lay.total,
               SIPA_EWORKSPACE, "%d key splits need a 256-byte aligned workspace of %lld bytes (have %lld)", nsplit,
               (long long)lay.total, (long long)p->workspace_bytes);
    SIPA_CHECK((int64_t)nsplit * shape.nc * 16 * D * 4 <= 0x7fffffff, SIPA_EINVAL, "split state too large");
  }
  PrefillArgs a;
  a.q = p->q;
  a.q_st = p->q_stride_t;
  a.q_sh = p->q_stride_h;
  a.k = p->k_cache;
  a.v = p->v_cache;
  a.kv_sh = p->kv_stride_h;
  a.kv_sn = p->kv_stride_n;
  a.bt = p->block_tables;
  a.bt_ss = p->bt_stride_s;
  a.bt_w = p->bt_width;
  a.ctx = p->context_lens;
  a.qstart = p->query_starts;
  a.qlen = p->query_lens;
  a.out = p->out;
  a.o_st = p->out_stride_t;
  a.o_sh = p->out_stride_h;
  a.S = S;
  a.G = G;
  a.qtiles = qtiles;
  a.npair = S * Hkv;
  a.tt = tt;
  a.T = p->num_tokens;
  a.nb = p->num_blocks;
  a.max_ctx = p->max_context;
  a.scale_log2 = p->scale * 1.4426950408889634f;
  a.nsplit = nsplit;
  a.chunk = chunk;
  a.ks = p->k_scale;
  a.vs = p->v_scale;
  a.ks_f32 = p->k_scale_dtype == SIPA_F32;
  a.vs_f32 = p->v_scale_dtype == SIPA_F32;
  {
    const int per16 = a.ks_f32 ? 4 : 8;  // scales per 16 bytes
    a.ks_vec = aligned16p(p->k_scale) && p->ks_stride_h % per16 == 0 && p->ks_stride_n % per16 == 0;
  }
  a.ks_sh = p->ks_stride_h;
  a.ks_sn = p->ks_stride_n;
  a.vs_sh = p->vs_stride_h;
  a.vs_sn = p->vs_stride_n;
  a.stage = (const uint16_t*)p->stage;
  a.st_sh = p->st_stride_h;
  a.st_sn = p->st_stride_n;
  a.st_sb = p->st_stride_b;
  a.n_stage = p->num_stage;
  a.tails = p->tail_slots;
  SIPA_CHECK(p->merge_path == SIPA_MERGE_AUTO || p->merge_path == SIPA_MERGE_MEMORY, SIPA_EINVAL,
             "merge_path %d is neither SIPA_MERGE_AUTO nor SIPA_MERGE_MEMORY", p->merge_path);
  a.mem_merge = p->merge_path == SIPA_MERGE_MEMORY;
  char* ws = (char*)p->workspace;
  a.counters = nsplit > 1 ? (int*)(ws + lay.counters) : nullptr;
  a.pm = nsplit > 1 ? (float*)(ws + lay.pm) : nullptr;
  a.pl = nsplit > 1 ? (float*)(ws + lay.pl) : nullptr;
  a.part = nsplit > 1 ? (float*)(ws + lay.part) : nullptr;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)wgs);
  // Key tiles: 64 keys at head_dim 64 (one barrier, one max reduction and one rescale test per 64 keys: four
  // 2048-token prompts 94 -> 84 us), 32 at head_dim 128, whose registers would otherwise halve the waves per SIMD
  // (166 -> 221 us). Tiles in flight (NPRE) within the register budget.
  if (D == 64) {
    if (shape.kh == 2) launch_prefill<64, 2, 64, 1, 8, 2>(mode, grid, st, a);
    else if (shape.nc == 16) launch_prefill<64, 2, 64, 1, 16, 1>(mode, grid, st, a);
    else if (shape.cw == 1) launch_prefill<64, 2, 64, 1, 8, 1>(mode, grid, st, a);
    else launch_prefill<64, 2, 64, 2, 8, 1>(mode, grid, st, a);
  } else {
    if (shape.kh == 2) launch_prefill<128, 2, 32, 1, 8, 2>(mode, grid, st, a);
    else if (shape.nc == 16) launch_prefill<128, 2, 32, 1, 16, 1>(mode, grid, st, a);
    else if (shape.cw == 1) launch_prefill<128, 2, 32, 1, 8, 1>(mode, grid, st, a);
    else launch_prefill<128, 2, 32, 2, 8, 1>(mode, grid, st, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIPA_EHIP, "prefill launch failed: %s", hipGetErrorString(e));
  return SIPA_OK;
}
