// Paged-attention decode for gfx950: one query token per sequence, K/V read in place from the block pool.
//
// Reference: engine/triton_decode.py:51-161 (_decode_kernel, _combine_kernel) and :188-238 (the wrapper).
//
// Work decomposition. A workgroup (4 waves) owns one (sequence s, KV head h, split sp): tokens
// [sp*chunk, min((sp+1)*chunk, ctx[s])). Splits past a sequence's end exit at once, so one grid
// (splits, Hkv, S) serves ragged batches: a long sequence spreads over many CUs, a short one uses one
// workgroup. Every query head of the GQA group is computed from the same K/V loads, so each KV head's cache
// is read from HBM once per call. The four waves of a workgroup take 32- (MFMA) or 64-token (VALU) tiles
// round-robin and merge their online-softmax states through LDS at the end. A workgroup that holds a whole
// sequence writes the output; otherwise it writes an unnormalised partial (acc, m, l) and either the last
// workgroup of the (s, h) to finish merges all partials (an atomic counter per (s, h)), or a separate combine
// kernel does.
//
// Online softmax per query head (reference engine/triton_decode.py:118-131), with scores kept in the exp2
// domain (x * scale * log2 e):  m' = max(m, max_t s_t);  a = 2^(m - m');  l = l a + sum_t 2^(s_t - m');
// acc = acc a + sum_t 2^(s_t - m') v_t;  out = acc / l.  Combine (reference :144-161):
// M = max_j m_j;  out = sum_j 2^(m_j - M) acc_j / sum_j 2^(m_j - M) l_j.
//
// MFMA kernel (bf16 q and pool, 16-token blocks, head_dim 64 or 128, group <= 16). Per 32-token tile (two
// blocks) and wave:
//   S^T[16 tok x 16 g] = K[16 tok x 32 d] . Q^T[32 d x 16 g]   v_mfma_f32_16x16x32_bf16, D/32 steps per block
//     A = K straight from HBM: lane (r, q4) = (lane % 16, lane / 16) loads 16 B of token r at channel
//     32 j + 8 q4, so the 16 lanes of a quarter-wave read 16 rows x 16 B and each load instruction covers one
//     contiguous 64-B half of every 128-B row of the block.
//     B = the group's query rows (zero rows pad G to 16), loaded once per wave.
//   Lane (r, q4) then holds head g = r for tokens 4 q4 .. 4 q4 + 3 of each block: the softmax state of head g
//   lives in the 4 lanes r, r+16, r+32, r+48 (two xor-shuffles give the tile max).
//   O^T[16 d x 16 g] += V^T[16 d x 32 tok] . P^T[32 tok x 16 g]    D/16 MFMAs per tile
//     B = P^T comes from the S^T registers without any shuffle (token slot i of lane q4 is token
//     16 (i / 4) + 4 q4 + i % 4); A = V^T needs 8 tokens of one channel per lane, so each wave stages its V
//     tile in LDS (coalesced 2 KiB block loads, row-major with padding) and reads it back transposed.
//   P enters the MFMA as two bf16 terms, P = P_hi + P_lo with P_hi = bf16(p) and P_lo = bf16(p - P_hi), two
//   MFMAs per d-tile on the same V operand: about 16 significant bits of P, where the reference keeps P in fp32
//   and runs P.V in TF32 (11 bits, engine/triton_decode.py:14-18,206-210); one bf16 term (8 bits) is the PHL =
//   false variant, selectable for measurement. The softmax itself and all accumulation stay fp32.
//
// VALU kernel (any supported shape, fp32 or bf16, all KV modes): lane = token for q.k (q of the group in
// LDS as fp32, fp32 FMAs), lane = channel for p.v (p of the tile in LDS). IEEE fp32 arithmetic throughout,
// as the reference uses for fp32 caches (engine/triton_decode.py:208-210).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <cstddef>
#include <mutex>
#include <vector>

#include "decode_common.h"

namespace sipa {

// Bytes of the bf16 kernel's leading scalar arguments (three pointers and six int32), before its DecodeArgs.
constexpr int kHotArgBytes = 3 * 8 + 6 * 4;

// NB: tiles in flight per wave (the register prefetch ring); PHL: P as a bf16 hi + lo pair (else one bf16 term).
template <int D, int NB, bool PHL>
__global__ void __launch_bounds__(kThreads) decode_mfma_bf16(const int32_t* __restrict__ hbt,
                                                             const int32_t* __restrict__ hctx,
                                                             const int32_t* __restrict__ hitems, int32_t hbt_ss,
                                                             int32_t hSH, int32_t hS, int32_t hchunk,
                                                             int32_t hmax_ctx, int32_t hbt_w, const DecodeArgs a) {
  constexpr int KS = D / 32;  // QK k-steps per block
  constexpr int DT = D / 16;  // PV d-tiles
  constexpr int VC = D / 32;  // 16-byte V chunks per lane per block
  constexpr int VP = MfmaSmem<D>::kVPitch;
  constexpr int CPR = D / 8;  // 16-byte chunks per token row
  __shared__ __align__(16) char smem[MfmaSmem<D>::kBytes];
  __shared__ int bids[kMaxSplitBlocks];  // this split's block ids
  __shared__ int last_flag;

  const HotArgs hp{hbt, hctx, hitems, hbt_ss, hSH, hS, hchunk, hmax_ctx, hbt_w};
  const WorkItem w = work_item(hp, a);
  const int sp = w.sp, h = w.h, s = w.s;
  const int start = w.start;
  const int G = a.G;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;

  // Prologue: the split's block ids, the context length, the query and the kernel arguments the first tiles need
  // are all requested before anything waits, so the first K/V loads follow one memory round trip.
  int ids[kIdsPerThread];
  fetch_split_ids_flat(hp.bt, hp.bt_ss, hp.bt_w, s, start, w.end, ids);
  const uint16_t* const kbase = (const uint16_t*)a.k;
  const uint16_t* const vbase = (const uint16_t*)a.v;
  const int64_t kv_sh = a.kv_sh, kv_sn = a.kv_sn;
  const int nblocks = a.nb;
  int ctx_raw;
  {
    // Every 64-byte line of the kernel arguments goes into the scalar cache in this same wait: the arguments the
    // epilogue reads are otherwise fetched after the barrier, and the first tile's LDS read of its block id (counted
    // with scalar loads) would wait for them.
    static_assert(kHotArgBytes + sizeof(DecodeArgs) <= 6 * 64 && kHotArgBytes + sizeof(DecodeArgs) >= 0x144,
                  "the six line loads stay inside the explicit kernel arguments");
    // The context length is loaded in the same block: the compiler waits for every outstanding scalar load before
    // an inline asm statement, so a load of its own would be one more round trip.
    const auto ka = __builtin_amdgcn_kernarg_segment_ptr();
    const int32_t* ctx_p = hp.ctx + s;
    uint32_t l0, l1, l2, l3, l4, l5;
    asm volatile(
        "s_load_dword %0, %8, 0x0\n"
        "s_load_dword %1, %7, 0x0\n"
        "s_load_dword %2, %7, 0x40\n"
        "s_load_dword %3, %7, 0x80\n"
        "s_load_dword %4, %7, 0xc0\n"
        "s_load_dword %5, %7, 0x100\n"
        "s_load_dword %6, %7, 0x140\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(ctx_raw), "=&s"(l0), "=&s"(l1), "=&s"(l2), "=&s"(l3), "=&s"(l4), "=&s"(l5)
        : "s"(ka), "s"(ctx_p), "s"(kbase), "s"(vbase), "s"(kv_sh), "s"(kv_sn), "s"(nblocks)
        : "memory");
  }
  const int ctx = min(ctx_raw, hp.max_ctx);  // as context_len()
  // The query group as the QK B operand. Lanes of padding heads (r >= G) load head G - 1 again: their score
  // columns run the same softmax as that head's and are never stored.
  bf16x8 qop[KS];
  {
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)s * a.q_ss + (int64_t)(h * G + min(r, G - 1)) * a.q_sh;
#pragma unroll
    for (int j = 0; j < KS; ++j) qop[j] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qrow + 32 * j + 8 * q4));
  }
  const bool past_end = w.nvalid < 0 && start >= ctx;  // grid: a split past this sequence's end
  const int end = max(start, min(w.end, ctx));
  const int nvalid = w.nvalid < 0 ? (ctx + hp.chunk - 1) / hp.chunk : w.nvalid;
  commit_split_ids_flat(ids, bids, nblocks);
  __syncthreads();  // block ids staged
  if (past_end) return;

  const uint16_t* kh = kbase + (int64_t)h * kv_sh;
  const uint16_t* vh = vbase + (int64_t)h * kv_sh;
  uint16_t* vw = (uint16_t*)smem + wave * 32 * VP;
  const int tr_off = tr16_offset(r, q4, VP);
  const int ntile = (end - start + 31) >> 5;
  const int mine = ntile > wave ? (ntile - wave + kWaves - 1) / kWaves : 0;  // tiles wave, wave + 4, ...

  auto tile_t0 = [&](int k) { return start + 32 * (wave + kWaves * k); };
  // Branch-free: a tile's second block past the split's end re-reads the first block (its rows are masked), so
  // the number of loads in flight is the same on every path and the compiler's wait counts can leave the
  // other ring slots outstanding.
  auto load_tile = [&](int k, KVTile<D>& tl) {
    const int t0 = tile_t0(k);
    const int bi = (t0 - start) >> 4;
    const int b0 = bids[bi];
    const int b1 = (t0 + 16 < end) ? bids[bi + 1] : b0;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int blk = mt ? b1 : b0;
      const uint16_t* kb = kh + (int64_t)blk * kv_sn;
      const uint16_t* vb = vh + (int64_t)blk * kv_sn;
#pragma unroll
      for (int j = 0; j < KS; ++j) tl.k[mt][j] = stream_load(kb + r * D + 32 * j + 8 * q4);
#pragma unroll
      for (int i = 0; i < VC; ++i) tl.v[mt][i] = stream_load(vb + 8 * (lane + 64 * i));
    }
  };

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Online softmax with a lazily updated max: scores are exponentiated against m_run, which is raised (and acc, l
  // rescaled) only when some head's tile max exceeds it by more than 2^8; until then p <= 256, which fp32 acc/l
  // and bf16 P hold without loss of relative precision, and the final acc / l is unchanged.
  constexpr float kRescaleSlack = 8.f;
  auto process_tile = [&](int t0, KVTile<D>& tl) {
    const bool partial = t0 + 32 > end;  // wave-uniform
    if (partial) {  // V rows at or past the end are zeroed so that 0-weight garbage cannot give NaN
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < VC; ++i)
          if (t0 + 16 * mt + (lane + 64 * i) / CPR >= end) tl.v[mt][i] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < VC; ++i) {
        const int c = lane + 64 * i;
        *(u32x4*)(vw + (16 * mt + c / CPR) * VP + (c % CPR) * 8) = tl.v[mt][i];
      }

    f32x4 sc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      sc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KS; ++j)
        sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, tl.k[mt][j]), qop[j], sc[mt], 0,
                                                         0, 0);
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
    mx *= a.scale_log2;  // raw scores -> exp2 domain (scale > 0 keeps the order)
    if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescaleSlack)) {  // rare after the first tile
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      m_run = m_new;
    }
    bf16x8 pop, plo;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = fast_exp2(fmaf(sc[i >> 2][i & 3], a.scale_log2, -m_run));
      psum += p;
      pop[i] = (__bf16)p;
      if (PHL) plo[i] = (__bf16)(p - (float)pop[i]);  // the rounding residual, exact in fp32
    }
    l_run += psum;

    wave_sync();  // the wave's V tile is in LDS
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const bf16x8 vop = read_v_operand<bf16x8>(vw, tr_off, VP, 16 * dt);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop, acc[dt], 0, 0, 0);
      if (PHL) acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, plo, acc[dt], 0, 0, 0);
    }
    wave_sync();  // reads done before the next tile overwrites the LDS tile
  };

  KVTile<D> ring[NB];
  if (mine >= 2 * NB) {
    // Pipelined: NB tiles in flight; in the steady state every consumed slot is refilled unconditionally.
#pragma unroll
    for (int j = 0; j < NB; ++j) load_tile(j, ring[j]);
    int k0 = 0;
    for (; k0 + 2 * NB <= mine; k0 += NB) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        process_tile(tile_t0(k0 + j), ring[j]);
        load_tile(k0 + j + NB, ring[j]);
      }
    }
    // Drain: tiles k0 .. k0 + NB - 1 are loaded, fewer than NB more remain.
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      process_tile(tile_t0(k0 + j), ring[j]);
      if (k0 + j + NB < mine) load_tile(k0 + j + NB, ring[j]);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (k0 + NB + j < mine) process_tile(tile_t0(k0 + NB + j), ring[j]);
  } else if (NB == 2 && mine > 0) {
    // Short split (1 to 3 tiles a wave) at the default depth: the tiles' loads in flight together, one path per
    // tile count so that no load is repeated and the compiler's waits are exact. (One tile at a time cost a memory
    // round trip per tile: C3's short work-list items 28.56 -> 28.15 us.)
    load_tile(0, ring[0]);
    if (mine == 1) {
      process_tile(tile_t0(0), ring[0]);
    } else {
      load_tile(1, ring[1 % NB]);
      process_tile(tile_t0(0), ring[0]);
      if (mine == 3) {
        load_tile(2, ring[0]);
        process_tile(tile_t0(1), ring[1 % NB]);
        process_tile(tile_t0(2), ring[0]);
      } else {
        process_tile(tile_t0(1), ring[1 % NB]);
      }
    }
  } else if (mine > 0) {
    // Short split at other depths (fewer than 2 NB tiles a wave): NB tiles in flight as well. Every slot's load is
    // issued (a load past the wave's last tile re-reads that tile), and each processed slot is refilled with the
    // tile NB ahead while one can remain, so that along the chain of tiles the compiler's waits count the loads
    // exactly and leave the younger slots outstanding.
#pragma unroll
    for (int j = 0; j < NB; ++j) load_tile(min(j, mine - 1), ring[j]);
    // tile k nested in tile k - 1's branch (compile-time k, so the ring stays in registers)
    auto short_tile = [&](auto self, auto kc) -> void {
      constexpr int k = decltype(kc)::value;
      if constexpr (k < 2 * NB - 1) {
        if (k < mine) {  // wave-uniform
          process_tile(tile_t0(k), ring[k % NB]);
          if constexpr (k + NB < 2 * NB - 1) load_tile(min(k + NB, mine - 1), ring[k % NB]);
          self(self, std::integral_constant<int, k + 1>());
        }
      }
    };
    short_tile(short_tile, std::integral_constant<int, 0>());
  }

  mfma_epilogue<D, false>(a, s, h, sp, nvalid, m_run, l_run, acc, smem, &last_flag);
}

// ---- VALU kernel: any supported shape, fp32 / bf16, KV modes 0 / 1 / 2 -----------------------------------------

template <int TQ>
__device__ __forceinline__ void load8_f32(const void* base, int64_t i, float (&f)[8]) {
  if (TQ == SIPA_F32) {
    const float4* p = (const float4*)((const float*)base + i);
    const float4 a = p[0], b = p[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const uint4 u = *(const uint4*)((const uint16_t*)base + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f[2 * k] = __uint_as_float(w[k] << 16);
      f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  }
}

__device__ __forceinline__ void load8_i8(const int8_t* p, float (&f)[8]) {
  const uint2 u = *(const uint2*)p;
  const uint32_t w[2] = {u.x, u.y};
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int b = 0; b < 4; ++b) f[4 * k + b] = (float)(int8_t)(w[k] >> (8 * b));
}

__device__ __forceinline__ float load_scale(const void* p, int64_t i, int is_f32) {
  return is_f32 ? ((const float*)p)[i] : f16_bits_to_f32(((const uint16_t*)p)[i]);
}

template <int D>
struct ValuSmem {
  static constexpr int kPBytes = kWaves * 64 * kMaxGroup * 4;  // per-wave p tiles [64 tok][16 g]
  static constexpr int kMergeBytes = (2 * kWaves * kMaxGroup + kWaves * kMaxGroup * D) * 4;
  static constexpr int kBytes = kPBytes > kMergeBytes ? kPBytes : kMergeBytes;
};

template <int TQ, int MODE, int D>
__global__ void __launch_bounds__(kThreads) decode_valu(const DecodeArgs a) {
  constexpr int DPL = (D + 63) / 64;  // channels per lane in p.v
  __shared__ __align__(16) float qs[kMaxGroup * D];
  __shared__ __align__(16) char smem[ValuSmem<D>::kBytes];
  __shared__ int last_flag;

  const WorkItem w = work_item(a);
  const int sp = w.sp, h = w.h, s = w.s;
  const int ctx = context_len(a, s);
  const int start = w.start;
  if (w.nvalid < 0 && start >= ctx) return;  // grid: a split past this sequence's end
  const int end = max(start, min(w.end, ctx));
  const int nvalid = w.nvalid < 0 ? splits_holding(ctx, a.chunk, a.chunk_old, a.n_old) : w.nvalid;
  const int G = a.G, B = a.B;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;

  for (int idx = threadIdx.x; idx < G * D; idx += kThreads)
    qs[idx] = load_as_f32(a.q, (int64_t)s * a.q_ss + (int64_t)(h * G + idx / D) * a.q_sh + idx % D, TQ);
  __syncthreads();

  const int32_t* btr = a.bt + (int64_t)s * a.bt_ss;
  const int n_quant = (ctx / B) * B;  // MODE 2: tokens in full (quantized) blocks; the rest are staged
  const int tail = (MODE == 2) ? tail_slot(a, s) : 0;
  float* pw = (float*)smem + wave * 64 * kMaxGroup;

  float m_run[kMaxGroup], l_run[kMaxGroup], acc[kMaxGroup][DPL];
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) {
    m_run[g] = kNegInf;
    l_run[g] = 0.f;
#pragma unroll
    for (int u = 0; u < DPL; ++u) acc[g][u] = 0.f;
  }

  for (int t0 = start + 64 * wave; t0 < end; t0 += 64 * kWaves) {
    const int t = t0 + lane;
    const bool valid = t < end;
    int blk = 0, off = 0;
    float sc[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) sc[g] = 0.f;
    float vscale = 1.f;
    if (valid) {
      blk = min(max(btr[min(t / B, a.bt_w - 1)], 0), a.nb - 1);
      off = t % B;
      const int64_t row = (int64_t)h * a.kv_sh + (int64_t)blk * a.kv_sn + (int64_t)off * D;
      const bool staged = (MODE == 2) && (t >= n_quant) && (tail >= 0);  // -1: no staging slot to read
      for (int d0 = 0; d0 < D; d0 += 8) {
        float kf[8];
        if (MODE == 0) {
          load8_f32<TQ>(a.k, row + d0, kf);
        } else if (staged) {
          load8_f32<SIPA_BF16>(a.stage, (int64_t)h * a.st_sh + (int64_t)tail * a.st_sn + (int64_t)off * a.st_sb + d0,
                               kf);
        } else {
          load8_i8((const int8_t*)a.k + row + d0, kf);
          if (MODE == 2) {
            const int64_t si = (int64_t)h * a.ks_sh + (int64_t)blk * a.ks_sn + d0;
#pragma unroll
            for (int i = 0; i < 8; ++i) kf[i] *= load_scale(a.ks, si + i, a.ks_f32);
          }
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
          if (g < G) {
            const float4 qa = *(const float4*)(qs + g * D + d0);
            const float4 qb = *(const float4*)(qs + g * D + d0 + 4);
            float x = sc[g];
            x = fmaf(qa.x, kf[0], x); x = fmaf(qa.y, kf[1], x); x = fmaf(qa.z, kf[2], x); x = fmaf(qa.w, kf[3], x);
            x = fmaf(qb.x, kf[4], x); x = fmaf(qb.y, kf[5], x); x = fmaf(qb.z, kf[6], x); x = fmaf(qb.w, kf[7], x);
            sc[g] = x;
          }
        }
      }
      if (MODE == 1) {
        const float ks = load_scale(a.ks, (int64_t)h * a.ks_sh + (int64_t)blk * a.ks_sn + off, a.ks_f32);
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) sc[g] *= ks;
      }
      if (MODE != 0) vscale = load_scale(a.vs, (int64_t)h * a.vs_sh + (int64_t)blk * a.vs_sn + off, a.vs_f32);
    }
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      if (g < G) {
        const float x = valid ? sc[g] * a.scale_log2 : kNegInf;
        const float m_new = fmaxf(m_run[g], wave_max(x));
        const float alpha = fast_exp2(m_run[g] - m_new);
        const float p = fast_exp2(x - m_new);
        l_run[g] = l_run[g] * alpha + p;
        m_run[g] = m_new;
#pragma unroll
        for (int u = 0; u < DPL; ++u) acc[g][u] *= alpha;
        pw[lane * kMaxGroup + g] = p * vscale;  // V's per-token scale folds into p; l keeps the unscaled p
      }
    }
    wave_sync();
    const int ntok = min(64, end - t0);
    for (int j = 0; j < ntok; ++j) {
      const int bj = __builtin_amdgcn_readlane(blk, j);
      const int oj = __builtin_amdgcn_readlane(off, j);
      const int64_t row = (int64_t)h * a.kv_sh + (int64_t)bj * a.kv_sn + (int64_t)oj * D;
      float vf[DPL];
#pragma unroll
      for (int u = 0; u < DPL; ++u) {
        const int d = lane + 64 * u;
        if (d < D)
          vf[u] = (MODE == 0) ? load_as_f32(a.v, row + d, TQ) : (float)((const int8_t*)a.v)[row + d];
        else
          vf[u] = 0.f;
      }
      const float4* prow = (const float4*)(pw + j * kMaxGroup);
#pragma unroll
      for (int g4 = 0; g4 < kMaxGroup / 4; ++g4) {
        if (4 * g4 < G) {
          const float4 p4 = prow[g4];
          const float pg[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int u = 0; u < DPL; ++u) acc[4 * g4 + e][u] = fmaf(pg[e], vf[u], acc[4 * g4 + e][u]);
        }
      }
    }
    wave_sync();
  }

  float lw[kMaxGroup];
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) lw[g] = (g < G) ? wave_sum(l_run[g]) : 0.f;
  __syncthreads();  // p tiles are dead: the LDS becomes the merge buffer
  float* ms = (float*)smem;
  float* ls = ms + kWaves * kMaxGroup;
  float* accs = ls + kWaves * kMaxGroup;
  if (lane < kMaxGroup) {
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
      if (g == lane) {
        ms[wave * kMaxGroup + g] = m_run[g];
        ls[wave * kMaxGroup + g] = lw[g];
      }
  }
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g)
    if (g < G)
#pragma unroll
      for (int u = 0; u < DPL; ++u) {
        const int d = lane + 64 * u;
        if (d < D) accs[(wave * kMaxGroup + g) * D + d] = acc[g][u];
      }
  __syncthreads();
  finish_split<D, TQ == SIPA_F32>(a, s, h, sp, nvalid, ms, ls, accs, &last_flag);
}

// ---- separate combine kernel ------------------------------------------------------------------------------------

template <int D, bool OUT_F32>
__global__ void __launch_bounds__(kThreads) combine_splits(const DecodeArgs a) {
  const int h = blockIdx.x, s = blockIdx.y;
  const int nvalid = splits_holding(context_len(a, s), a.chunk, a.chunk_old, a.n_old);
  if (nvalid <= 1) return;  // the single split wrote the output itself
  combine_group<D, OUT_F32, kMergePlain>(a, s, h, nvalid);
}

// ---- host side --------------------------------------------------------------------------------------------------

static int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

struct WorkspaceLayout {
  int64_t counters, pm, pl, part, total;
};

static WorkspaceLayout workspace_layout(int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t splits) {
  WorkspaceLayout w;
  w.counters = 0;
  w.pm = kCounterBytes;
  w.pl = w.pm + align256(S * Hq * splits * 4);
  w.part = w.pl + align256(S * Hq * splits * 4);
  w.total = w.part + align256(S * Hq * splits * D * 4);
  return w;
}

static int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// At most one workgroup per CU: each workgroup pays a fixed cost of two dependent memory round trips before its
// first tile and the split merge after its last, so a few long-running workgroups beat many short ones (measured
// on MI355X, bf16 32 x 8192: 4 splits 27.9 us, 8 splits 29.2 us, 16 splits 44.6 us). A small batch does not fill
// the chip either: past 8 splits every 8 more add a round trip to the merge, so splits stay at 512 tokens or more
// unless a short context fits 8 splits of at least 128 (bf16, 2 KV heads: 1 x 1024 best at 8 splits, 6.3 us
// against 6.9 at 4; 1 x 8192 at 16, 9.8 against 10.3 at 32; 4 x 8192 at 16, 10.9 against 12.8 at 32; 8 x 4096
// at 8, 10.4 against 11.5 at 16). The INT8 kernels, two workgroups per CU, take splits down to 256 tokens past 8
// splits (1 x 4096: 9.8 us at 16 splits against 11.6 at 8; 1 x 1024: 7.6 us at 8 against 8.6 at 4). kMaxChunk
// spreads a long sequence of a full grid over several CUs.
int choose_splits_host(int S, int Hkv, int max_ctx, int cu_count, bool int8) {
  if (S <= 0 || Hkv <= 0 || max_ctx <= 0) return 1;
  if (cu_count <= 0) cu_count = 256;
  const int64_t programs = (int64_t)S * Hkv;
  int64_t splits = (cu_count + programs - 1) / programs;
  const int64_t most = std::max<int64_t>(ceil_div(max_ctx, int8 ? kMinChunk : kLatencyChunk),
                                         std::min<int64_t>(kShortSplits, ceil_div(max_ctx, kShortChunk)));
  splits = std::min<int64_t>(splits, most);
  splits = std::max<int64_t>(splits, ceil_div(max_ctx, kMaxChunk));
  return (int)std::max<int64_t>(1, std::min<int64_t>(splits, 1 << 20));
}

int split_chunk_host(int max_ctx, int splits) {
  splits = std::max(1, splits);
  const int per = ceil_div(std::max(1, max_ctx), splits);
  // A split never exceeds the block ids the MFMA kernel stages in LDS (kMaxSplitBlocks blocks of 16 tokens).
  return std::min(ceil_div(per, kChunkAlign) * kChunkAlign, kMaxSplitBlocks * 16);
}

template <typename Kernel>
static int launch(Kernel k, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k, grid, dim3(kThreads), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIPA_EHIP, "decode launch failed: %s", hipGetErrorString(e));
  return SIPA_OK;
}

template <int TQ, int D>
static int launch_valu(int mode, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  switch (mode) {
    case 0: return launch(decode_valu<TQ, 0, D>, grid, a, st);
    case 1: return launch(decode_valu<TQ, 1, D>, grid, a, st);
    default: return launch(decode_valu<TQ, 2, D>, grid, a, st);
  }
}

template <int TQ>
static int dispatch_valu(int D, int mode, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  switch (D) {
    case 16: return launch_valu<TQ, 16>(mode, grid, a, st);
    case 32: return launch_valu<TQ, 32>(mode, grid, a, st);
    case 64: return launch_valu<TQ, 64>(mode, grid, a, st);
    default: return launch_valu<TQ, 128>(mode, grid, a, st);
  }
}

template <bool F32>
static int dispatch_combine(int D, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  switch (D) {
    case 16: return launch(combine_splits<16, F32>, grid, a, st);
    case 32: return launch(combine_splits<32, F32>, grid, a, st);
    case 64: return launch(combine_splits<64, F32>, grid, a, st);
    default: return launch(combine_splits<128, F32>, grid, a, st);
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Tiles each wave keeps in flight in the MFMA kernel: 2 (C2 at 4 splits: 26.2 us, against 26.5 us with 3 or 4).
// SIPA_PREFETCH_TILES, read once per process, overrides it for tuning sweeps.
static int prefetch_tiles(int D) {
  (void)D;
  static const int env = [] {
    const char* e = getenv("SIPA_PREFETCH_TILES");
    return e ? atoi(e) : 0;
  }();
  return env > 0 ? env : 2;
}

// The bf16 kernel takes its prologue's fields as leading scalars (preloaded into SGPRs), then the whole block.
template <int D, int NB, bool PHL>
static int launch_bf16(dim3 grid, const DecodeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((decode_mfma_bf16<D, NB, PHL>), grid, dim3(kThreads), 0, st, a.bt, a.ctx, a.items, (int32_t)a.bt_ss,
                     a.S * a.Hkv, a.S, a.chunk, a.max_ctx, a.bt_w, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIPA_EHIP, "decode launch failed: %s", hipGetErrorString(e));
  return SIPA_OK;
}

template <bool PHL>
static int launch_mfma(int D, int nb, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  if (D == 64) {
    switch (nb) {
      case 1: return launch_bf16<64, 1, PHL>(grid, a, st);
      case 2: return launch_bf16<64, 2, PHL>(grid, a, st);
      case 3: return launch_bf16<64, 3, PHL>(grid, a, st);
      default: return launch_bf16<64, 4, PHL>(grid, a, st);
    }
  }
  switch (nb) {
    case 1: return launch_bf16<128, 1, PHL>(grid, a, st);
    case 2: return launch_bf16<128, 2, PHL>(grid, a, st);
    default: return launch_bf16<128, 3, PHL>(grid, a, st);
  }
}

}  // namespace sipa

using namespace sipa;

extern "C" int32_t sipa_choose_splits(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context,
                                      int32_t cu_count) {
  return choose_splits_host(num_seqs, num_kv_heads, max_context, cu_count, false);
}

extern "C" int32_t sipa_split_chunk(int32_t max_context, int32_t num_splits) {
  return split_chunk_host(max_context, num_splits);
}

// The INT8 kernels run two workgroups per CU and stage at most kMaxInt8Split tokens of scales per split.
extern "C" int32_t sipa_choose_splits_for(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context,
                                          int32_t cu_count, int32_t kv_mode) {
  const bool int8 = kv_mode != SIPA_KV_PLAIN;
  const int cu = cu_count > 0 ? cu_count : sipa_device_cu_count(-1);
  int splits = choose_splits_host(num_seqs, num_kv_heads, max_context, (int8 ? 2 : 1) * cu, int8);
  if (int8 && max_context > 0) splits = std::max(splits, ceil_div(max_context, kMaxInt8Split));
  return splits;
}

// Grids of exactly two workgroups per CU, each CU holding workgroups L and L + CUs (the dispatcher deals the first
// CU-count workgroups one per CU, then the next ones): the older of each pair wins instruction-issue arbitration
// and streams faster while both run (C4, equal splits: 17.5 against 23 us to the end of streaming), so the older
// class gets splits `ratio` times as long. This needs sequences x KV heads to divide the CU count (the first
// CUs / SH splits of every pair are then the older class). Default ratio: kOldSplitRatio; SIPA_OLD_RATIO, read once
// per process, overrides it for tuning sweeps (<= 1: equal splits).
constexpr double kOldSplitRatio = 1.6;

static double old_split_ratio() {
  static const double r = [] {
    const char* e = getenv("SIPA_OLD_RATIO");
    return e ? atof(e) : kOldSplitRatio;
  }();
  return r;
}

static void two_class_splits(int64_t SH, int max_ctx, int splits, int cu, int max_split, int* chunk, int* chunk_old,
                             int* n_old) {
  *n_old = 0;
  *chunk_old = 0;
  const double r = old_split_ratio();
  if (r <= 1.0 || cu <= 0 || SH <= 0 || cu % SH != 0 || splits != 2 * (cu / SH)) return;
  const int n = (int)(cu / SH);
  constexpr int kAlign = 32 * kWaves;  // whole 32-token tiles for every wave of the MFMA kernels
  const int co = ceil_div((int64_t)std::ceil(r * max_ctx / (n * (1.0 + r))), kAlign) * kAlign;
  if (co > max_split || (int64_t)n * co >= max_ctx) return;
  const int cy = ceil_div(ceil_div(max_ctx - (int64_t)n * co, n), kAlign) * kAlign;
  if (cy > co) return;
  *n_old = n;
  *chunk_old = co;
  *chunk = cy;
}

// int8: the INT8 kernels' splits are at most kMaxInt8Split tokens (more splits than requested if need be).
static int resolve_splits(int S, int Hkv, int max_ctx, int requested, bool int8, int* chunk) {
  int splits = requested;
  if (splits <= 0) splits = sipa_choose_splits_for(S, Hkv, max_ctx, 0, int8 ? SIPA_KV_INT8_TOKEN : SIPA_KV_PLAIN);
  if (int8) splits = std::max(splits, ceil_div(max_ctx, kMaxInt8Split));
  *chunk = split_chunk_host(max_ctx, splits);
  return ceil_div(max_ctx, *chunk);  // no split that is empty for every sequence
}

extern "C" int32_t sipa_decode_split_grid(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context,
                                          int32_t num_splits, int32_t kv_mode, int32_t* chunk, int32_t* chunk_old,
                                          int32_t* n_old) {
  SIPA_CHECK(num_seqs > 0 && num_kv_heads > 0 && max_context > 0 && kv_mode >= 0 && kv_mode <= 2 && chunk &&
                 chunk_old && n_old,
             SIPA_EINVAL, "split grid: bad arguments");
  int c = 0, co = 0, no = 0;
  const int splits = resolve_splits(num_seqs, num_kv_heads, max_context, num_splits, kv_mode != SIPA_KV_PLAIN, &c);
  if (splits > 1 && kv_mode == SIPA_KV_INT8_KCHAN)
    two_class_splits((int64_t)num_seqs * num_kv_heads, max_context, splits, sipa_device_cu_count(-1), kMaxInt8Split,
                     &c, &co, &no);
  *chunk = c;
  *chunk_old = co;
  *n_old = no;
  return splits;
}

extern "C" int32_t sipa_build_work_list(const int32_t* ctx, int32_t S, int32_t Hkv, int32_t cu_count,
                                        int32_t items_per_cu, int32_t max_piece, int32_t* items, int32_t capacity,
                                        int32_t* max_splits) {
  SIPA_CHECK(ctx != nullptr && S >= 0 && Hkv > 0, SIPA_EINVAL, "work list: bad arguments");
  if (cu_count <= 0) cu_count = 256;
  if (items_per_cu <= 0) items_per_cu = 2;
  const int64_t cap = max_piece > 0 ? std::min<int64_t>(max_piece, kMaxSplitBlocks * 16) : kMaxSplitBlocks * 16;
  SIPA_CHECK(cap >= kMinChunk, SIPA_EINVAL, "max_piece %d < %d", max_piece, kMinChunk);
  int64_t total = 0;
  for (int s = 0; s < S; ++s) {
    SIPA_CHECK(ctx[s] >= 1, SIPA_EINVAL, "context length %d of sequence %d < 1", ctx[s], s);
    total += ctx[s];
  }
  total *= Hkv;
  int64_t piece = (total + (int64_t)cu_count * items_per_cu - 1) / ((int64_t)cu_count * items_per_cu);
  // The smallest piece: 512 tokens (small ragged batches, bf16: a 16,000-token sequence of 8 cut into 256-token
  // pieces merged 63 partials, 15.1 us, into 512-token ones 32, 12.3 us); 256 for the INT8 kernels, which pass
  // their 4096-token cap (their small batches: 10.5 us at 256 against 12.1 at 512).
  const int min_piece = (max_piece > 0 && max_piece <= kMaxInt8Split) ? kMinChunk : kLatencyChunk;
  piece = std::min<int64_t>(std::max<int64_t>((piece + kChunkAlign - 1) / kChunkAlign * kChunkAlign, min_piece),
                            cap / kChunkAlign * kChunkAlign);
  struct Item {
    int32_t s, h, sp, n, start, end;
  };
  std::vector<Item> v;
  int32_t maxn = 1;
  for (int s = 0; s < S; ++s) {
    // near-equal pieces of the pair, each a multiple of 64 tokens (block- and tile-aligned starts)
    const int64_t n0 = (ctx[s] + piece - 1) / piece;
    const int64_t per = ((ctx[s] + n0 - 1) / n0 + kChunkAlign - 1) / kChunkAlign * kChunkAlign;
    const int32_t n = (int32_t)((ctx[s] + per - 1) / per);
    maxn = std::max(maxn, n);
    for (int h = 0; h < Hkv; ++h)
      for (int k = 0; k < n; ++k)
        v.push_back(Item{s, h, k, n, (int32_t)(k * per), (int32_t)std::min<int64_t>((k + 1) * per, ctx[s])});
  }
  SIPA_CHECK(v.size() <= 0x7fffffff, SIPA_EINVAL, "work list too long");
  if (max_splits) *max_splits = maxn;
  if (items == nullptr) return (int32_t)v.size();
  SIPA_CHECK((int64_t)v.size() <= capacity, SIPA_EINVAL, "work list of %d items exceeds capacity %d",
             (int)v.size(), capacity);
  std::stable_sort(v.begin(), v.end(), [](const Item& x, const Item& y) { return x.end - x.start > y.end - y.start; });
  for (size_t i = 0; i < v.size(); ++i) {
    int32_t* o = items + 8 * i;
    o[0] = v[i].s, o[1] = v[i].h, o[2] = v[i].sp, o[3] = v[i].n, o[4] = v[i].start, o[5] = v[i].end;
    o[6] = o[7] = 0;
  }
  return (int32_t)v.size();
}

extern "C" int32_t sipa_check_work_list(const int32_t* items, int32_t n, int32_t S, int32_t Hkv, int32_t max_ctx,
                                        int32_t num_splits) {
  SIPA_CHECK(items != nullptr && n >= 0 && S >= 0 && Hkv > 0 && max_ctx > 0, SIPA_EINVAL, "work list: bad arguments");
  struct Entry {
    int64_t pair;
    int32_t sp, ns, start, end, index;
  };
  std::vector<Entry> e((size_t)n);
  for (int i = 0; i < n; ++i) {
    const int32_t* it = items + 8 * (int64_t)i;
    const int32_t s = it[0], h = it[1], sp = it[2], ns = it[3], st = it[4], en = it[5];
    SIPA_CHECK(s >= 0 && s < S && h >= 0 && h < Hkv, SIPA_EINVAL, "work item %d: pair (%d, %d) out of range", i, s, h);
    SIPA_CHECK(ns >= 1 && ns <= num_splits && sp >= 0 && sp < ns, SIPA_EINVAL,
               "work item %d: split %d of %d (num_splits %d)", i, sp, ns, num_splits);
    SIPA_CHECK(st >= 0 && st < en && en <= max_ctx && en - st <= kMaxSplitBlocks * 16, SIPA_EINVAL,
               "work item %d: tokens [%d, %d) outside [0, %d) or longer than %d", i, st, en, max_ctx,
               kMaxSplitBlocks * 16);
    e[i] = Entry{(int64_t)s * Hkv + h, sp, ns, st, en, i};
  }
  std::sort(e.begin(), e.end(), [](const Entry& x, const Entry& y) {
    return x.pair != y.pair ? x.pair < y.pair : x.sp < y.sp;
  });
  // Within a pair (sorted by split): splits 0, 1, ..., ns - 1 exactly once, one stated ns, ranges in order.
  for (size_t k = 0; k < e.size(); ++k) {
    const bool first = k == 0 || e[k].pair != e[k - 1].pair;
    const int expect = first ? 0 : e[k - 1].sp + 1;
    SIPA_CHECK(e[k].sp == expect && (first || e[k].ns == e[k - 1].ns), SIPA_EINVAL,
               "work item %d: pair (%lld, %lld) lists split %d where split %d (of %d stated) is due", e[k].index,
               (long long)(e[k].pair / Hkv), (long long)(e[k].pair % Hkv), e[k].sp, expect, e[k].ns);
    SIPA_CHECK(first || e[k].start >= e[k - 1].end, SIPA_EINVAL, "work item %d: overlaps split %d of its pair",
               e[k].index, e[k - 1].sp);
    const bool last = k + 1 == e.size() || e[k + 1].pair != e[k].pair;
    SIPA_CHECK(!last || e[k].sp == e[k].ns - 1, SIPA_EINVAL, "pair (%lld, %lld): %d splits stated, %d listed",
               (long long)(e[k].pair / Hkv), (long long)(e[k].pair % Hkv), e[k].ns, e[k].sp + 1);
  }
  return SIPA_OK;
}

extern "C" int64_t sipa_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                                               int32_t head_dim, int32_t num_splits) {
  if (num_splits <= 1) return 0;
  return workspace_layout(num_seqs, num_q_heads, num_kv_heads, head_dim, num_splits).total;
}

// ---- the allocation-free entry point's split workspace -----------------------------------------------------------

// sipa_decode_noalloc keeps its split partials and merge counters here: a file-scope device array, one copy per GPU
// the library runs on, held until the process ends. In host code the name is only a handle for
// hipGetSymbolAddress; every host use goes through the per-device address scratch_on_current_device() returns.
constexpr int64_t kScratchBytes = 16ll << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

__global__ void __launch_bounds__(256) zero_words(int32_t* p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}

static std::mutex g_scratch_lock;
static void* g_scratch_ptr[64];  // per device: the array's address, NULL until that device's first call

static int zero_scratch_counters(void* ptr, hipStream_t st) {
  hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, st, (int32_t*)ptr, kMaxCounters);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIPA_EHIP, "clearing the scratch counters: %s", hipGetErrorString(e));
  return SIPA_OK;
}

// The scratch array of the current device. Its first call on a device looks up the array's address and zeroes the
// merge-counter region with a fill kernel on `st` (a kernel, not a memset, so that a first call under stream capture
// records a kernel node); later calls reuse both. reset: zero the counters again on every call.
static int scratch_on_current_device(hipStream_t st, char** out, bool reset = false) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SIPA_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
  SIPA_CHECK(dev >= 0 && dev < 64, SIPA_EUNSUPPORTED, "device %d: the allocation-free entry serves devices 0..63", dev);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(SIPA_EHIP, "address of the scratch array on device %d: %s", dev, hipGetErrorString(e));
    const int rc = zero_scratch_counters(ptr, st);
    if (rc != SIPA_OK) return rc;
    g_scratch_ptr[dev] = ptr;
  } else if (reset) {
    const int rc = zero_scratch_counters(g_scratch_ptr[dev], st);
    if (rc != SIPA_OK) return rc;
  }
  *out = (char*)g_scratch_ptr[dev];
  return SIPA_OK;
}

extern "C" int32_t sipa_decode_noalloc_reset(void* stream) {
  char* base = nullptr;
  return scratch_on_current_device((hipStream_t)stream, &base, true);
}

static int decode_impl(const sipa_decode_params* p, void* stream, bool use_scratch);

extern "C" int32_t sipa_decode(const sipa_decode_params* p, void* stream) { return decode_impl(p, stream, false); }

extern "C" int32_t sipa_decode_noalloc(const sipa_decode_params* p, void* stream) {
  return decode_impl(p, stream, true);
}

static int decode_impl(const sipa_decode_params* p, void* stream, bool use_scratch) {
  SIPA_CHECK(p != nullptr, SIPA_EINVAL, "params is NULL");
  SIPA_CHECK(p->struct_size == (int32_t)sizeof(sipa_decode_params), SIPA_EINVAL,
             "struct_size %d does not match this library's sipa_decode_params (%d bytes, ABI %d)", p->struct_size,
             (int)sizeof(sipa_decode_params), SIPA_ABI_VERSION);
  const int S = p->num_seqs, Hq = p->num_q_heads, Hkv = p->num_kv_heads, D = p->head_dim, B = p->block_size;
  if (S == 0) return SIPA_OK;
  SIPA_CHECK(S > 0 && S <= 65535, SIPA_EINVAL, "num_seqs %d outside [0, 65535]", S);
  SIPA_CHECK(Hkv > 0 && Hkv <= 65535 && Hq > 0 && Hq % Hkv == 0, SIPA_EINVAL,
             "num_q_heads %d must be a positive multiple of num_kv_heads %d", Hq, Hkv);
  const int G = Hq / Hkv;
  SIPA_CHECK(G <= kMaxGroup, SIPA_EUNSUPPORTED, "GQA group %d > %d", G, kMaxGroup);
  SIPA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, SIPA_EUNSUPPORTED, "head_dim %d not in {16,32,64,128}", D);
  SIPA_CHECK(p->scale > 0.f && p->scale < __builtin_inff(), SIPA_EINVAL,
             "scale %g must be positive and finite (the kernels take maxima of the unscaled scores)", (double)p->scale);
  SIPA_CHECK(B > 0 && 64 % B == 0, SIPA_EINVAL, "block_size %d must divide 64 (block-aligned 64-token tiles)", B);
  SIPA_CHECK(p->max_context > 0, SIPA_EINVAL, "max_context %d must be >= 1", p->max_context);
  SIPA_CHECK(p->num_blocks > 0, SIPA_EINVAL, "num_blocks %d must be >= 1", p->num_blocks);
  SIPA_CHECK(p->bt_stride_s >= 0 && p->bt_stride_s <= INT32_MAX, SIPA_EINVAL,
             "block_tables row stride %lld outside [0, 2^31)", (long long)p->bt_stride_s);
  SIPA_CHECK(p->bt_width > 0 && (int64_t)p->bt_width * B >= p->max_context, SIPA_EINVAL,
             "block_tables rows of %d entries cannot cover max_context %d (block size %d)", p->bt_width,
             p->max_context, B);
  SIPA_CHECK(p->q_dtype == SIPA_F32 || p->q_dtype == SIPA_BF16, SIPA_EUNSUPPORTED, "q_dtype %d not f32/bf16",
             p->q_dtype);
  SIPA_CHECK(p->kv_mode >= 0 && p->kv_mode <= 2, SIPA_EINVAL, "kv_mode %d", p->kv_mode);
  SIPA_CHECK(p->q && p->k_cache && p->v_cache && p->block_tables && p->context_lens && p->out, SIPA_EINVAL,
             "NULL tensor pointer");
  SIPA_CHECK(aligned16(p->k_cache) && aligned16(p->v_cache), SIPA_EINVAL, "K/V pools must be 16-byte aligned");
  SIPA_CHECK(p->kv_stride_h % 16 == 0 && p->kv_stride_n % 16 == 0, SIPA_EINVAL,
             "pool head/block strides must be multiples of 16 elements");
  const int mode = p->kv_mode;
  if (mode != SIPA_KV_PLAIN) {
    SIPA_CHECK(p->k_scale && p->v_scale, SIPA_EINVAL, "INT8 modes need k_scale and v_scale");
    SIPA_CHECK((p->k_scale_dtype == SIPA_F16 || p->k_scale_dtype == SIPA_F32) &&
                   (p->v_scale_dtype == SIPA_F16 || p->v_scale_dtype == SIPA_F32),
               SIPA_EUNSUPPORTED, "scales must be f16 or f32");
  }
  if (mode == SIPA_KV_INT8_KCHAN) {
    SIPA_CHECK(p->stage && p->tail_slots && p->num_stage > 0, SIPA_EINVAL,
               "int8 per-channel K needs stage, tail_slots and num_stage >= 1");
    SIPA_CHECK(aligned16(p->stage) && p->st_stride_h % 8 == 0 && p->st_stride_n % 8 == 0 && p->st_stride_b % 8 == 0,
               SIPA_EINVAL, "staging must be 16-byte aligned with strides multiple of 8");
  }

  const int n_items = p->num_items;
  SIPA_CHECK(n_items >= 0, SIPA_EINVAL, "num_items %d < 0", n_items);
  int chunk = 0, splits = 1;
  if (n_items > 0) {
    SIPA_CHECK(p->work_items != nullptr && aligned16(p->work_items), SIPA_EINVAL,
               "work_items must be a 16-byte aligned device array");
    SIPA_CHECK(p->num_splits >= 1, SIPA_EINVAL, "with a work list, num_splits must be its largest split count");
    splits = p->num_splits;
  } else {
    splits = resolve_splits(S, Hkv, p->max_context, p->num_splits, mode != SIPA_KV_PLAIN, &chunk);
  }
  SIPA_CHECK((int64_t)(Hq / Hkv) * splits * D * 4 < INT32_MAX, SIPA_EUNSUPPORTED,
             "%d splits: a KV head's partial rows exceed 2 GiB", splits);

  DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.q = p->q;
  a.q_ss = p->q_stride_s;
  a.q_sh = p->q_stride_h;
  a.k = p->k_cache;
  a.v = p->v_cache;
  a.kv_sh = p->kv_stride_h;
  a.kv_sn = p->kv_stride_n;
  a.bt = p->block_tables;
  a.bt_ss = p->bt_stride_s;
  a.ctx = p->context_lens;
  a.out = p->out;
  a.o_ss = p->out_stride_s;
  a.o_sh = p->out_stride_h;
  a.ks = p->k_scale;
  a.ks_sh = p->ks_stride_h;
  a.ks_sn = p->ks_stride_n;
  a.vs = p->v_scale;
  a.vs_sh = p->vs_stride_h;
  a.vs_sn = p->vs_stride_n;
  a.stage = p->stage;
  a.st_sh = p->st_stride_h;
  a.st_sn = p->st_stride_n;
  a.st_sb = p->st_stride_b;
  a.tail = p->tail_slots;
  a.ks_f32 = p->k_scale_dtype == SIPA_F32;
  a.vs_f32 = p->v_scale_dtype == SIPA_F32;
  a.S = S;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = G;
  a.B = B;
  a.splits = splits;
  a.chunk = chunk;
  a.max_ctx = p->max_context;
  a.nb = p->num_blocks;
  a.bt_w = p->bt_width;
  a.n_stage = mode == SIPA_KV_INT8_KCHAN ? p->num_stage : 1;
  a.items = n_items > 0 ? p->work_items : nullptr;
  a.fused = n_items > 0 || p->combine == SIPA_COMBINE_FUSED;  // a work list always merges in place
  a.scale_log2 = p->scale * 1.4426950408889634f;

  hipStream_t st = (hipStream_t)stream;
  if (splits > 1) {
    SIPA_CHECK((int64_t)S * Hkv <= kMaxCounters, SIPA_EINVAL,
               "%lld (sequence, KV head) pairs exceed the %d merge counters of a split launch", (long long)S * Hkv,
               kMaxCounters);
    const WorkspaceLayout w = workspace_layout(S, Hq, Hkv, D, splits);
    char* base = nullptr;
    if (use_scratch) {
      SIPA_CHECK(w.total <= kScratchBytes, SIPA_EWORKSPACE,
                 "%d splits of %d sequences x %d query heads need a %lld-byte workspace; the allocation-free entry "
                 "holds %lld (use sipa_decode with a workspace, or fewer splits)", splits, S, Hq, (long long)w.total,
                 (long long)kScratchBytes);
      const int rc = scratch_on_current_device(st, &base);
      if (rc != SIPA_OK) return rc;
    } else {
      SIPA_CHECK(p->workspace != nullptr && p->workspace_bytes >= w.total, SIPA_EWORKSPACE,
                 "workspace of %lld bytes needed for %d splits (got %lld)", (long long)w.total, splits,
                 (long long)p->workspace_bytes);
      SIPA_CHECK(((uintptr_t)p->workspace & 255) == 0, SIPA_EWORKSPACE, "workspace must be 256-byte aligned");
      base = (char*)p->workspace;
    }
    a.counters = (int32_t*)(base + w.counters);
    a.pm = (float*)(base + w.pm);
    a.pl = (float*)(base + w.pl);
    a.part = (float*)(base + w.part);
  }

  // The MFMA kernels: bf16 query, 16-token blocks, head_dim 64 / 128, 16-byte aligned rows, and for INT8 pools
  // fp16 scales laid out for 8-byte (per-token) and 16-byte (per-channel) vector loads.
  const bool q_aligned = aligned16(p->q) && p->q_stride_s % 8 == 0 && p->q_stride_h % 8 == 0;
  bool mfma_ok = p->q_dtype == SIPA_BF16 && B == 16 && (D == 64 || D == 128) && q_aligned;
  int int8_variant = 0;
  if (mfma_ok && mode != SIPA_KV_PLAIN) {
    auto tok_scales_ok = [](const void* ptr, int dt, int64_t sh, int64_t sn) {
      return dt == SIPA_F16 && ((uintptr_t)ptr & 7) == 0 && sh % 4 == 0 && sn % 4 == 0;
    };
    const bool vs_ok = tok_scales_ok(p->v_scale, p->v_scale_dtype, p->vs_stride_h, p->vs_stride_n);
    if (mode == SIPA_KV_INT8_TOKEN) {
      int8_variant = 1;
      mfma_ok = vs_ok && tok_scales_ok(p->k_scale, p->k_scale_dtype, p->ks_stride_h, p->ks_stride_n);
    } else if (p->ks_stride_n == 0) {
      int8_variant = 3;
      mfma_ok = vs_ok;
    } else {
      int8_variant = 2;
      mfma_ok = vs_ok && p->k_scale_dtype == SIPA_F16 && aligned16(p->k_scale) && p->ks_stride_h % 8 == 0 &&
                p->ks_stride_n % 8 == 0;
    }
  }
  const bool valu_stream = p->impl == SIPA_IMPL_VALU_STREAM || p->impl == SIPA_IMPL_VALU_DOT2;
  if (valu_stream) {
    const bool tok_scales = mode == SIPA_KV_PLAIN ||
                            (mode == SIPA_KV_INT8_TOKEN && p->k_scale_dtype == SIPA_F16 && p->v_scale_dtype == SIPA_F16);
    SIPA_CHECK(p->q_dtype == SIPA_BF16 && B == 16 && q_aligned && tok_scales &&
                   valu_stream_supported(D, G, mode, p->impl == SIPA_IMPL_VALU_DOT2),
               SIPA_EUNSUPPORTED, "the VALU streaming kernels need a bf16 query, block 16, head_dim 64/128, a group "
               "of 6-8, a bf16 pool or an int8 per-token pool with fp16 scales, and 16-byte aligned rows");
  }
  SIPA_CHECK(p->impl != SIPA_IMPL_MFMA_PBF16 || (mfma_ok && mode == SIPA_KV_PLAIN), SIPA_EUNSUPPORTED,
             "the bf16-P MFMA variant needs a bf16 query and pool, block 16, head_dim 64/128, 16-byte aligned rows");
  SIPA_CHECK(p->impl != SIPA_IMPL_MFMA || mfma_ok, SIPA_EUNSUPPORTED,
             "the MFMA kernels need a bf16 query, block 16, head_dim 64/128, 16-byte aligned rows and fp16 scales "
             "(or fp32 channel scales with a zero block stride)");
  const bool p_bf16 = p->impl == SIPA_IMPL_MFMA_PBF16;
  const bool use_mfma = mfma_ok && (p->impl == SIPA_IMPL_AUTO || p->impl == SIPA_IMPL_MFMA || p_bf16);

  // Measured on C4 (sweeps of the ratio, alternating runs): format B 30.9 -> 30.1 us at 1.6; the per-token format
  // within noise at every ratio (and 0.2 us slower at 1.6 with its workgroup-wide scale staging), so it keeps equal
  // splits, as does the bf16 kernel, whose policy grid is one workgroup per CU.
  if (n_items == 0 && use_mfma && splits > 1 && mode == SIPA_KV_INT8_KCHAN)
    two_class_splits((int64_t)S * Hkv, p->max_context, splits, sipa_device_cu_count(-1), kMaxInt8Split, &a.chunk,
                     &a.chunk_old, &a.n_old);
  const int64_t wgs = n_items > 0 ? (int64_t)n_items : (int64_t)S * Hkv * splits;
  SIPA_CHECK(wgs <= 0x7fffffff, SIPA_EINVAL, "%lld workgroups exceed the grid limit", (long long)wgs);
  const dim3 grid((unsigned)wgs);
  int rc;
  if (valu_stream)
    rc = launch_valu_stream(D, G, mode, p->impl == SIPA_IMPL_VALU_DOT2, grid, a, st);
  else if (use_mfma && mode == SIPA_KV_PLAIN)
    rc = p_bf16 ? launch_mfma<false>(D, prefetch_tiles(D), grid, a, st)
                : launch_mfma<true>(D, prefetch_tiles(D), grid, a, st);
  else if (use_mfma)
    rc = launch_mfma_int8(D, int8_variant, prefetch_tiles(D), grid, a, st);
  else if (p->q_dtype == SIPA_F32)
    rc = dispatch_valu<SIPA_F32>(D, mode, grid, a, st);
  else
    rc = dispatch_valu<SIPA_BF16>(D, mode, grid, a, st);
  if (rc != SIPA_OK || splits == 1 || a.fused) return rc;
  return p->q_dtype == SIPA_F32 ? dispatch_combine<true>(D, dim3(Hkv, S), a, st)
                                : dispatch_combine<false>(D, dim3(Hkv, S), a, st);
}
