// Paged decode over INT8 K/V pools on the matrix cores (gfx950), dequantization fused into the operands.
//
// Reference: engine/triton_decode.py:93-117,126-130 (KV_MODE 1 and 2) and engine/quant_cache.py (the formats):
//   mode 1 (format "int8"): K and V int8 [Hkv, N, B, D], fp16 scales per token [Hkv, N, B] each;
//   mode 2 (format "int8-kchannel"): K int8 with fp16 scales per (block, channel) [Hkv, N, D] (a zero block stride
//     gives one scale per (head, channel)), each sequence's partial last block of K in a bf16 staging slot;
//     V as in mode 1.
// Same work decomposition, prefetch ring, online softmax and split merge as the bf16 kernel (decode.hip); the
// differences are the operands, per 16-token block (one MFMA M-tile):
//   S^T = K_int . Q^T on v_mfma_f32_16x16x32_f16. int8 codes become fp16 exactly (the byte, biased by 128, is
//     placed under the exponent of 1024 with v_perm_b32, then 1152 is subtracted); the bf16 query is exact in
//     fp16 over fp16's normal range. Mode 1 multiplies the fp32 scores by the per-token K scale, as the reference
//     does (score_t = (q . k_int_t) s_t). Mode 2 folds the block's channel scales into the query instead,
//     Q' = q * s_c, carried as two fp16 operands (an exact high part and a low part, relative error about 2^-14,
//     two MFMAs per k-step): one fp16 rounding of Q' (2^-11) is too coarse when outlier channels make the q.k
//     terms large and the softmax peaked. The staged partial block uses v_mfma_f32_16x16x32_bf16 with the bf16
//     query and bf16 staged K (exact products).
//   O^T += V_int^T . P'^T on the fp16 MFMA with the per-token V scale folded into P (P' = p s_v, fp16), as the
//     reference does (acc += (p s_v) v_int; l keeps the unscaled p). The V tile goes to LDS already converted to
//     fp16 and is read back transposed. The reference forms P' in fp32 (engine/triton_decode.py:126-130); fp16
//     has its 11 significant bits but not its exponent range: with small V scales (V absmax under about 0.05)
//     most P' would fall into fp16 subnormals. Each wave therefore takes p' = p 2^e, with 2^e chosen from the
//     largest V scale of its tokens so that max(s_v) 2^e lies in [2^10, 2^11): P' = p' s_v <= 2^4 2^11 stays
//     below fp16's 65504, and every term within 2^-29 of the largest stays normal. The factor rides on the exp2's
//     offset (p' = 2^(x - (m - e))), so l and acc both carry it and the wave reports its max as m - e: the merges
//     and the final acc / l are exactly those of p.
// Lane (r, q4) loads 16-byte pieces 64 j + 16 q4 of K row r (one load instruction covers 64 contiguous bytes of each
// of 16 rows), so the query operand uses that channel order too: k-slot 8 jj + i of lane group q4 is channel
// 64 (jj / 2) + 16 q4 + 8 (jj % 2) + i.
#include "decode_common.h"

namespace sipa {

// 4 int8 codes (one 32-bit word) -> 4 fp16 values, exact.
__device__ __forceinline__ void codes_to_f16(uint32_t w, f16x2& lo, f16x2& hi) {
  const uint32_t u = w ^ 0x80808080u;  // code + 128 in each byte
  const f16x2 bias = {(_Float16)1152.f, (_Float16)1152.f};
  lo = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
  hi = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
}

__device__ __forceinline__ f16x8 codes8_to_f16(uint32_t w0, uint32_t w1) {
  f16x2 a, b, c, d;
  codes_to_f16(w0, a, b);
  codes_to_f16(w1, c, d);
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ float h2f(uint32_t bits16) { return f16_bits_to_f32(bits16 & 0xffffu); }

template <int D>
struct Int8Tile {
  u32x4 k[2][D / 64];   // K codes: lane (r, q4) holds token r's channels (D/4) q4 .. (D/4)(q4+1)
  u32x4 v[2][D / 64];   // V codes as 16-byte row chunks
  uint32_t kc[2];       // mode 2: one 32-bit word (2 fp16 channel scales) of the block's D scales per lane
};

// Per-token scales (K in mode 1, V in every mode) live in LDS, loaded in the prologue with one 16-byte load per half
// block row: a tile then issues only its eight 16-byte code loads. (Per-tile 8-byte scale loads made a third of the
// load instructions for 1.5% of the bytes, and load issue, not bytes, limited the kernel.) Each block's 16 fp16
// scales are 8 words. Two stagings:
// - per wave (modes 2 and 3, V scales only): each wave stages only the blocks its own tiles cover, in a region of its
//   own: lane l holds block 2 (wave + 4 (l / 2)) + l % 2 of the split (tile l / 2 of the wave), loaded after the ids
//   are staged and before the wave's first tile loads, and the wave syncs with itself alone, so it starts on its
//   first tile when that tile is in. With the workgroup-wide staging below, every wave waited for all of its
//   workgroup's first tiles (512 workgroups issue 32 MiB at once; the first tile was processed ~8 us into the call):
//   C4(a) 31.9 -> 30.0 us.
// - per workgroup (mode 1, K and V scales): thread t loads block t's rows with the block id it fetched itself, before
//   the ids barrier, and the workgroup waits for all of them (and the first tiles) at one barrier. Per-wave staging
//   made mode 1 slower (C4(b) 27.8 -> 28.3 us, and 28.7 with a barrier restoring a common start).
constexpr int kScaleBlocks = kMaxInt8Split / 16;
constexpr int kWaveScaleBlocks = kScaleBlocks / kWaves;  // blocks of one wave's tiles in a split

// MODE 1: per-token K scales; 2: per-(block, channel) K scales; 3: mode 2 with one channel scale per (head,
// channel) for every block (a zero block stride), folded into the query once.
template <int D, int MODE, int NB>
__global__ void __launch_bounds__(kThreads, 2) decode_mfma_int8(const DecodeArgs a) {
  constexpr int KS = D / 32;   // QK k-steps per block
  constexpr int DT = D / 16;   // PV d-tiles
  constexpr int KL = D / 64;   // 16-byte K loads per lane per block
  constexpr int VC = D / 64;   // 16-byte V chunks (16 codes) per lane per block
  constexpr int VP = MfmaSmem<D>::kVPitch;
  constexpr int CPR = D / 16;  // 16-code chunks per token row

  __shared__ __align__(16) char smem[MfmaSmem<D>::kBytes];
  // mode 2: each wave's channel scales of two tiles (slot = tile index parity), [wave][slot][block][lane]
  __shared__ __align__(16) uint32_t kcs[(MODE == 2) ? kWaves * 2 * 2 * 64 : 1];
  constexpr int kScaleArrays = (MODE == 1) ? 2 : 1;                              // [V, K] or [V] token scales
  constexpr bool kWaveScales = MODE != 1;  // the token-scale staging (see kScaleBlocks)
  // [wave][arr][block of the wave][8] (kWaveScales) or [arr][block of the split][8]
  __shared__ __align__(16) uint32_t tsc[kScaleArrays * kScaleBlocks * 8];
  __shared__ __align__(8) int bids[kMaxInt8Split / 16];  // a split of at most kMaxInt8Split tokens
  __shared__ uint32_t vmax_bits[kWaves];  // per-workgroup staging: each wave's largest V scale (fp16 bits)
  __shared__ int last_flag;

  {
    // Each 64-byte line of the kernel arguments, requested at entry in one wait: the argument loads the compiler
    // places later (work item, block table, epilogue) then hit the scalar cache instead of each costing a round trip
    // (and the first tile's LDS reads, counted with scalar loads, do not wait behind them).
    static_assert(sizeof(DecodeArgs) <= 5 * 64 && sizeof(DecodeArgs) >= 0x104,
                  "the five line loads stay inside the kernel arguments");
    const auto ka = __builtin_amdgcn_kernarg_segment_ptr();
    uint32_t l0, l1, l2, l3, l4;
    asm volatile(
        "s_load_dword %0, %5, 0x0\n"
        "s_load_dword %1, %5, 0x40\n"
        "s_load_dword %2, %5, 0x80\n"
        "s_load_dword %3, %5, 0xc0\n"
        "s_load_dword %4, %5, 0x100\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(l0), "=&s"(l1), "=&s"(l2), "=&s"(l3), "=&s"(l4)
        : "s"(ka)
        : "memory");
  }
  const WorkItem w = work_item(a);
  const int sp = w.sp, h = w.h, s = w.s;
  const int start = w.start;
  const int G = a.G;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  // K codes: load j of lane (r, q4) is bytes 64 j + 16 q4 .. + 15 of row r, so that each load instruction covers 64
  // contiguous bytes of each of 16 rows; k-step jj of lane group q4 then holds channels kchan(jj) .. kchan(jj) + 7.
  auto kchan = [&](int jj) { return 64 * (jj >> 1) + 16 * q4 + 8 * (jj & 1); };

  const int wend = min(w.end, start + kMaxInt8Split);  // the host never makes longer splits; LDS holds no more
  // Prologue: the split's block ids, the query, the context length and staging slot, and every line of the kernel
  // arguments are requested before anything waits; the query's conversion runs after the first tiles' loads are
  // issued. The first K/V loads then follow one memory round trip.
  static_assert(kMaxInt8Split / 16 == kThreads, "one block id per thread");
  int ids[1];
  fetch_split_ids_flat(a.bt, a.bt_ss, a.bt_w, s, start, wend, ids);
  // The query group in bf16, channel order of the int8 K layout: k-step j of lane (r, q4) (zero for r >= G).
  const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)s * a.q_ss + (int64_t)(h * G + min(r, G - 1)) * a.q_sh;
  auto load_qb = [&](int j) {
    u32x4 u = *(const u32x4*)(qrow + kchan(j));
    if (r >= G) u = u32x4{0, 0, 0, 0};
    return __builtin_bit_cast(bf16x8, u);
  };
  u32x4 qraw[KS];
#pragma unroll
  for (int j = 0; j < KS; ++j) qraw[j] = *(const u32x4*)(qrow + kchan(j));
  int ctx_raw, tail_raw;
  {
    // The context length and staging slot in one wait (the compiler waits for every outstanding scalar load before
    // an inline asm statement, so separate loads would each cost a round trip).
    const int32_t* ctx_p = a.ctx + s;
    const int32_t* tail_p = MODE >= 2 ? a.tail + s : ctx_p;
    asm volatile(
        "s_load_dword %0, %2, 0x0\n"
        "s_load_dword %1, %3, 0x0\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(ctx_raw), "=&s"(tail_raw)
        : "s"(ctx_p), "s"(tail_p)
        : "memory");
  }
  const int ctx = min(ctx_raw, a.max_ctx);  // as context_len()
  const bool past_end = w.nvalid < 0 && start >= ctx;  // grid: a split past this sequence's end
  const int end = max(start, min(wend, ctx));
  const int nvalid = w.nvalid < 0 ? splits_holding(ctx, a.chunk, a.chunk_old, a.n_old) : w.nvalid;
  const int n_quant = (ctx >> 4) << 4;  // mode 2: tokens in full (quantized) blocks
  // staging slot of the partial last block, -1 if none (as tail_slot())
  const int tail = (MODE >= 2) ? min(tail_raw, a.n_stage - 1) : -1;
  const uint16_t* ksh = (const uint16_t*)a.ks + (int64_t)h * a.ks_sh;
  const uint16_t* vsh = (const uint16_t*)a.vs + (int64_t)h * a.vs_sh;
  // The token scales of one block (two 16-byte half rows per array) into sreg.
  u32x4 sreg[kScaleArrays][2];
  auto load_scales = [&](int64_t blk) {
#pragma unroll
    for (int arr = 0; arr < kScaleArrays; ++arr) {
      const uint16_t* base = arr ? ksh : vsh;
      const int64_t sn = arr ? a.ks_sn : a.vs_sn;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) sreg[arr][hf] = *(const u32x4*)(base + blk * sn + 8 * hf);
    }
  };
  // Per-workgroup staging: thread t's block t, with the id it fetched (threads past the split read its last block
  // again, not staged).
  if (!kWaveScales) load_scales(min(max(ids[0], 0), a.nb - 1));
  commit_split_ids_flat(ids, bids, a.nb);
  __syncthreads();
  if (past_end) return;
  const int nblk = (end - start + 15) >> 4;  // blocks of this split, <= kMaxInt8Split / 16
  // The block whose scales this thread stages: per wave, lane l's block of the wave's tiles (lanes past the split
  // read its last block again, never used), issued before the wave's first tile loads; per workgroup, block t.
  const int my_bi = kWaveScales ? 2 * (wave + kWaves * (lane >> 1)) + (lane & 1) : (int)threadIdx.x;
  if (kWaveScales) load_scales(bids[min(my_bi, nblk - 1)]);

  constexpr bool kconst = MODE == 3;  // one channel scale per (head, channel) for every block
  // qh: the query in fp16 (modes 1, 2), or the high part of Q' = q * s (mode 3) with ql its low part,
  // fp16(Q' - qh), so that qh + ql carries Q' to about 2^-22. A head whose largest |q| (|Q'| in mode 3) lies
  // outside [2^-6, 2^8) is first scaled by 2^-shift to bring it into [2^6, 2^7): fp16 then holds it without
  // overflow (|q| > 65504) or subnormal loss, and mode 2's q * s products keep headroom. The factor is exact and
  // the softmax scale of that head (lane column r) takes its inverse, so the scores equal unscaled ones bit for
  // bit wherever those are representable. Computed by convert_query() once the first tiles' loads are out.
  f16x8 qh[KS], ql[KS];
  int qshift = 0;
  float sl2 = a.scale_log2;
  float vshift = 0.f;  // p' = p 2^vshift (set once the wave's V scales are in)
  auto convert_query = [&]() {
    float qf[KS][8];
    float qmax = 0.f;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      u32x4 u = qraw[j];
      if (r >= G) u = u32x4{0, 0, 0, 0};
      const bf16x8 qb = __builtin_bit_cast(bf16x8, u);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qf[j][i] = (float)qb[i];
        if (kconst) {
          const int64_t ci = (int64_t)h * a.ks_sh + kchan(j) + i;
          qf[j][i] *= a.ks_f32 ? ((const float*)a.ks)[ci] : f16_bits_to_f32(((const uint16_t*)a.ks)[ci]);
        }
        qmax = fmaxf(qmax, fabsf(qf[j][i]));
      }
    }
    qmax = max_over_rows(qmax);  // head r over the four lane groups
    const int qexp = qmax > 0.f ? (int)((__float_as_uint(qmax) >> 23) & 0xff) - 127 : 0;  // floor(log2) of a normal
    qshift = (qexp >= 8 || qexp < -6) ? qexp - 6 : 0;
    sl2 = ldexpf(a.scale_log2, qshift);  // this lane's head: the softmax scale times 2^shift
#pragma unroll
    for (int j = 0; j < KS; ++j) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = ldexpf(qf[j][i], -qshift);
        qh[j][i] = (_Float16)x;
        ql[j][i] = (_Float16)(x - (float)qh[j][i]);
      }
    }
  };

  const int8_t* kh = (const int8_t*)a.k + (int64_t)h * a.kv_sh;
  const int8_t* vh = (const int8_t*)a.v + (int64_t)h * a.kv_sh;
  _Float16* vw = (_Float16*)smem + wave * 32 * VP;
  const int tr_off = tr16_offset(r, q4, VP);
  const int ntile = (end - start + 31) >> 5;
  const int mine = ntile > wave ? (ntile - wave + kWaves - 1) / kWaves : 0;
  auto tile_t0 = [&](int k) { return start + 32 * (wave + kWaves * k); };

  auto load_tile = [&](int k, Int8Tile<D>& tl) {
    const int t0 = tile_t0(k);
    const int bi = (t0 - start) >> 4;
    const int b0 = bids[bi];
    const int b1 = (t0 + 16 < end) ? bids[bi + 1] : b0;  // branch-free: a missing second block re-reads the first
    // Mode 2's channel scales first: the staging of the next tile's scales (stage_kc) then waits for them alone,
    // not for the tile's codes issued after them. Lane L holds channels 2L, 2L + 1 (lanes past D / 2 repeat).
    if (MODE == 2) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        tl.kc[mt] = *(const uint32_t*)(ksh + (int64_t)(mt ? b1 : b0) * a.ks_sn + 2 * (lane % (D / 2)));
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int64_t blk = mt ? b1 : b0;
      const int8_t* kb = kh + blk * a.kv_sn;
      const int8_t* vb = vh + blk * a.kv_sn;
#pragma unroll
      for (int j = 0; j < KL; ++j)
        tl.k[mt][j] = __builtin_nontemporal_load((const u32x4*)(kb + r * D + 64 * j + 16 * q4));
#pragma unroll
      for (int i = 0; i < VC; ++i) tl.v[mt][i] = __builtin_nontemporal_load((const u32x4*)(vb + 16 * (lane + 64 * i)));
    }
  };
  // Token scales of tokens 4 q4 .. 4 q4 + 3 of the tile's block mt. Per wave: tile t0 is the wave's tile
  // k = ((t0 - start) / 32 - wave) / kWaves, whose blocks lanes 2 k, 2 k + 1 staged; per workgroup: the split's
  // block (t0 - start) / 16 + mt. A second block past the end holds the split's last block: its tokens are masked.
  uint32_t* const tsw = tsc + (kWaveScales ? wave * kScaleArrays * kWaveScaleBlocks * 8 : 0);
  constexpr int kRegionBlocks = kWaveScales ? kWaveScaleBlocks : kScaleBlocks;
  auto token_scales = [&](int arr, int t0, int mt) {
    const int bl = kWaveScales ? 2 * ((((t0 - start) >> 5) - wave) >> 2) + mt : min(((t0 - start) >> 4) + mt, nblk - 1);
    return *(const uint2*)(tsw + (arr * kRegionBlocks + bl) * 8 + 2 * q4);
  };
  // p' = p 2^vshift: 2^vshift brings the largest V scale of the wave's tokens (per wave) or of the split's (per
  // workgroup) into [2^10, 2^11), or 1 when every scale is 0. Scales are non-negative fp16, whose bit patterns
  // order like their values.
  auto shift_of = [](uint32_t mb) {
    const float vm = h2f(mb);
    return vm > 0.f ? (float)(10 - ((int)((__float_as_uint(vm) >> 23) & 0xff) - 127)) : 0.f;
  };
  // This thread's block's scales into LDS and the wave's largest V scale among them. Per wave it is called where the
  // compiler can count the loads issued after the scale loads (inside each branch), so that the wait is exact.
  auto stage_scales = [&]() {
#pragma unroll
    for (int arr = 0; arr < kScaleArrays; ++arr)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        *(u32x4*)(tsw + (arr * kRegionBlocks + (kWaveScales ? lane : (int)threadIdx.x)) * 8 + 4 * hf) = sreg[arr][hf];
    const int nv = min(max(end - (start + 16 * my_bi), 0), 16);  // tokens of this thread's block in the split
    uint32_t mb = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t b = (sreg[0][j >> 3][(j >> 1) & 3] >> (16 * (j & 1))) & 0xffffu;
      if (j < nv) mb = max(mb, b);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, o));
    if (kWaveScales)
      vshift = shift_of(mb);
    else if (lane == 0)
      vmax_bits[wave] = mb;
  };

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // p <= 2^4 against the lazily raised max, so that P' = p 2^vshift s_v <= 2^4 2^11 stays within fp16.
  constexpr float kRescaleSlack = 4.f;
  // Mode 2: a tile's channel scales go through LDS (each lane then reads the 8 D / 32 it needs), into the wave's
  // slot of the tile's index parity. The pipelined loop stages tile k + 1's scales right after tile k, so a tile
  // starts with them in LDS; the short path stages them as it starts the tile.
  auto kc_slot = [&](int slot) { return kcs + (MODE == 2 ? (wave * 2 + slot) * 128 : 0); };
  auto stage_kc = [&](const Int8Tile<D>& tl, int slot) {
    if (MODE == 2) {
      uint32_t* w = kc_slot(slot);
      w[lane] = tl.kc[0];
      w[64 + lane] = tl.kc[1];
    }
  };
  auto process_tile = [&](int t0, Int8Tile<D>& tl, int slot, bool prestaged) {
    const bool partial = t0 + 32 > end;
    const uint32_t* kcw = kc_slot(slot);
    if (MODE == 2) {
      if (!prestaged) stage_kc(tl, slot);
      wave_sync();
    }
    // V codes -> fp16 -> LDS (rows at or past the end are zero).
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < VC; ++i) {
        const int c = lane + 64 * i;
        const int row = c / CPR;
        u32x4 wv = tl.v[mt][i];
        if (partial && t0 + 16 * mt + row >= end) wv = u32x4{0, 0, 0, 0};
        const f16x8 lo = codes8_to_f16(wv[0], wv[1]);
        const f16x8 hi = codes8_to_f16(wv[2], wv[3]);
        _Float16* dst = vw + (16 * mt + row) * VP + (c % CPR) * 16;
        *(f16x8*)dst = lo;
        *(f16x8*)(dst + 8) = hi;
      }

    f32x4 sc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      sc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int tb = t0 + 16 * mt;
      if (MODE >= 2 && tail >= 0 && tb == n_quant && tb < end) {
        // The sequence's partial last block: bf16 K from its staging slot, exact bf16 products.
        const uint16_t* st = (const uint16_t*)a.stage + (int64_t)h * a.st_sh + (int64_t)tail * a.st_sn +
                             (int64_t)r * a.st_sb;
#pragma unroll
        for (int j = 0; j < KS; ++j)
          sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, *(const u32x4*)(st + kchan(j))),
                                                           load_qb(j), sc[mt], 0, 0, 0);  // reloaded: rare
        if (qshift != 0) sc[mt] *= ldexpf(1.f, -qshift);  // the unscaled bf16 query: onto the head's scale
        continue;
      }
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const u32x4 kw = tl.k[mt][j >> 1];
        const f16x8 kop = codes8_to_f16(kw[2 * (j & 1)], kw[2 * (j & 1) + 1]);
        if (MODE == 1) {
          sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qh[j], sc[mt], 0, 0, 0);
        } else if (MODE == 3) {
          sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qh[j], sc[mt], 0, 0, 0);
          sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, ql[j], sc[mt], 0, 0, 0);
        } else {
          // Q' = q * s with the block's fp16 channel scales s, as an exact high part plus a low part: s_hi keeps
          // the top 3 significant bits of s (sign, exponent, 2 mantissa bits), so q * s_hi (8 x 3 bits) is exact
          // in fp16; the low part q * s - q_hi, one fused multiply-add (packed fp16), is q * (s - s_hi) rounded
          // once, relative to that small remainder only. (Written as q * (s - s_hi), the subtraction compiled to
          // unpacked fp16 subtracts and repacks: three instructions a pair.)
          const u32x4 cw = *(const u32x4*)(kcw + 64 * mt + kchan(j) / 2);
          const f16x8 s_all = __builtin_bit_cast(f16x8, cw);
          const f16x8 s_hi = __builtin_bit_cast(f16x8, cw & 0xff00ff00u);
          const f16x8 q_hi = qh[j] * s_hi;
          const f16x8 q_lo = __builtin_elementwise_fma(qh[j], s_all, -q_hi);
          sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, q_hi, sc[mt], 0, 0, 0);
          sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, q_lo, sc[mt], 0, 0, 0);
        }
      }
      if (MODE == 1) {
        const uint2 kw = token_scales(1, t0, mt);
        sc[mt][0] *= h2f(kw.x);
        sc[mt][1] *= h2f(kw.x >> 16);
        sc[mt][2] *= h2f(kw.y);
        sc[mt][3] *= h2f(kw.y >> 16);
      }
    }
    if (partial) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (t0 + 16 * mt + 4 * q4 + i >= end) sc[mt][i] = kNegInf;
    }
    float mx = vmax(vmax(vmax(sc[0][0], sc[0][1]), vmax(sc[0][2], sc[0][3])),
                    vmax(vmax(sc[1][0], sc[1][1]), vmax(sc[1][2], sc[1][3])));
    mx = max_over_rows(mx);
    mx *= sl2;
    if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      m_run = m_new;
    }
    f16x8 pop;
    float psum = 0.f;
    const uint2 vsc[2] = {token_scales(0, t0, 0), token_scales(0, t0, 1)};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int mt = i >> 2, e = i & 3;
      const float p = fast_exp2(fmaf(sc[mt][e], sl2, vshift - m_run));  // p 2^vshift
      psum += p;
      const uint32_t vsw = (e < 2) ? vsc[mt].x : vsc[mt].y;
      pop[i] = (_Float16)(p * h2f(vsw >> (16 * (e & 1))));
    }
    l_run += psum;

    wave_sync();  // the wave's V tile is in LDS
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const f16x8 vop = read_v_operand<f16x8>((const uint16_t*)vw, tr_off, VP, 16 * dt);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, acc[dt], 0, 0, 0);
    }
    wave_sync();
  };

  Int8Tile<D> ring[NB];
  const bool piped = mine >= 2 * NB;
  if (piped) {
#pragma unroll
    for (int j = 0; j < NB; ++j) load_tile(j, ring[j]);
    convert_query();
    if (kWaveScales) stage_scales();
  } else {
    convert_query();
    if (kWaveScales) stage_scales();
  }
  if (kWaveScales) {
    wave_sync();  // the wave's token scales are in its LDS region
  } else {
    stage_scales();
    __syncthreads();  // the split's token scales are staged
    uint32_t mb = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) mb = max(mb, vmax_bits[i]);
    vshift = shift_of(mb);
  }
  if (piped) {
    // Tile k is in ring[k % NB]; after tile k, tile k + 1's channel scales (mode 2) go to LDS slot (k + 1) & 1.
    stage_kc(ring[0], 0);
    int k0 = 0;
    for (; k0 + 2 * NB <= mine; k0 += NB) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int k = k0 + j;
        process_tile(tile_t0(k), ring[j], k & 1, true);
        load_tile(k + NB, ring[j]);
        stage_kc(ring[(j + 1) % NB], (k + 1) & 1);  // k + 1 < k0 + 2 NB <= mine
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = k0 + j;
      process_tile(tile_t0(k), ring[j], k & 1, true);
      if (k + NB < mine) load_tile(k + NB, ring[j]);
      if (k + 1 < mine) stage_kc(ring[(j + 1) % NB], (k + 1) & 1);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = k0 + NB + j;
      if (k < mine) {
        process_tile(tile_t0(k), ring[j], k & 1, true);
        if (k + 1 < mine) stage_kc(ring[(j + 1) % NB], (k + 1) & 1);
      }
    }
  } else {
    for (int k = 0; k < mine; ++k) {
      load_tile(k, ring[0]);
      process_tile(tile_t0(k), ring[0], 0, false);
    }
  }

  // l and acc carry 2^vshift: as the state of p they belong to the max m_run - vshift.
  mfma_epilogue<D, false>(a, s, h, sp, nvalid, m_run - vshift, l_run, acc, smem, &last_flag);
}

template <typename Kernel>
static int launch_int8(Kernel k, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k, grid, dim3(kThreads), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIPA_EHIP, "int8 decode launch failed: %s", hipGetErrorString(e));
  return SIPA_OK;
}

template <int D, int MODE>
static int launch_int8_depth(int nb, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  switch (nb) {
    case 1: return launch_int8(decode_mfma_int8<D, MODE, 1>, grid, a, st);
    case 2: return launch_int8(decode_mfma_int8<D, MODE, 2>, grid, a, st);
    default: return launch_int8(decode_mfma_int8<D, MODE, 3>, grid, a, st);
  }
}

// mode: 1, 2, or 3 (mode 2 with a zero block stride of the channel scales).
int launch_mfma_int8(int D, int mode, int nb, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  if (D == 64) {
    switch (mode) {
      case 1: return launch_int8_depth<64, 1>(nb, grid, a, st);
      case 2: return launch_int8_depth<64, 2>(nb, grid, a, st);
      default: return launch_int8_depth<64, 3>(nb, grid, a, st);
    }
  }
  switch (mode) {
    case 1: return launch_int8_depth<128, 1>(nb, grid, a, st);
    case 2: return launch_int8_depth<128, 2>(nb, grid, a, st);
    default: return launch_int8_depth<128, 3>(nb, grid, a, st);
  }
}

}  // namespace sipa
