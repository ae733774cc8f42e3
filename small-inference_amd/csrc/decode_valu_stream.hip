// Paged decode on the vector ALUs with the MFMA kernels' streaming structure: the A/B competitor of the matrix-core
// kernels (decode.hip decode_mfma_bf16, decode_int8.hip decode_mfma_int8). Same grid, split policy, block-id
// staging, NB-tile register prefetch ring of nontemporal 16-byte loads, lazy online softmax and split merge; only the
// dot products differ: here each lane computes them on the fp32 VALU with the query group in registers.
//
// Reference math: engine/triton_decode.py:93-131 (scores, online softmax; INT8 per-token K/V with the scales
// folded into the score and into p), engine/triton_decode.py:144-161 (the split combine).
//
// Lane layout per 16-token block: lane (r, q4) = (lane % 16, lane / 16) holds token r's channels
// c(j, i) = 4 CH j + CH q4 + i (j < KC, i < CH) of K and of V, loaded as KC 16-byte chunks, CH = 8 (bf16) or
// 16 (int8) channels per chunk: one load instruction covers a contiguous 64-byte piece of each of the block's 16
// rows, as in the MFMA kernels. A tile is two blocks (32 tokens), so a lane sees tokens r and 16 + r.
//   scores  s[t][g] = sum over the lane's D/4 channels, then over the 4 lanes q4 (two cross-row swaps);
//   softmax per head over the tile's 32 tokens: max over the two blocks, then over the 16 lanes r (four DPP steps);
//   P.V     acc[g][c] += p[t][g] v[t][c] for the lane's channels, summed over r only once, after the split.
// DOT = 0: fp32 FMAs (bf16 and int8 values converted to fp32). DOT = 1: v_dot2 pair products with fp32 accumulation
// (bf16 pairs for a bf16 pool, with P rounded to bf16 as in the bf16 MFMA kernel; fp16 pairs for int8 pools, with
// P' = p s_v rounded to fp16 as in the INT8 MFMA kernel); the P.V pairs are the same channel of the tile's two tokens.
// INT8 codes are used as c + 128 (unsigned bytes; exact in fp32, bf16 and fp16): the bias is removed once, from
// the score with the query's channel sums, and from the output with the sum of the p' weights.
#include "decode_common.h"

namespace sipa {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));

// All-reduce over the 16 lanes of a row (lanes r of one q4): butterfly with quad permutes and row mirrors.
template <bool MAX>
__device__ __forceinline__ float row16_reduce(float x) {
  auto op = [](float u, float v) { return MAX ? fmaxf(u, v) : u + v; };
  x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false)));
  x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false)));
  x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false)));
  x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false)));
  return x;
}

// byte k (0..3) of a dword as fp32 (v_cvt_f32_ubyte{k}).
__device__ __forceinline__ float ubyte_f32(uint32_t u, int k) { return (float)((u >> (8 * k)) & 0xffu); }

// byte k (0..3) of each of two dwords -> the fp16 pair (1024 + byte of w0, 1024 + byte of w1) (exact).
__device__ __forceinline__ half2_t bytes_to_f16_pair(uint32_t w0, uint32_t w1, int k) {
  // gather byte k of w0 and of w1 into the low bytes of one dword, then place 0x64 (the exponent of 1024) above each
  const uint32_t both = __builtin_amdgcn_perm(w1, w0, (uint32_t)(k | ((4 + k) << 8)) | 0x0c0c0000u);
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, both, 0x04010400u));
}

template <int D, int MODE>
struct ValuTile {
  static constexpr int KC = MODE == 0 ? D / 32 : D / 64;  // 16-byte chunks per lane per block
  u32x4 k[2][KC];
  u32x4 v[2][KC];
  uint32_t ks[2], vs[2];  // MODE 1: the per-token fp16 scales of tokens r and 16 + r (low 16 bits)
};

template <int D, int MODE, int DOT, int G, int NB>
__global__ void __launch_bounds__(kThreads) decode_valu_stream(const DecodeArgs a) {
  constexpr int CH = MODE == 0 ? 8 : 16;  // channels per 16-byte chunk
  constexpr int KC = D / (4 * CH);        // chunks per lane per block
  constexpr int CL = D / 4;               // channels per lane
  constexpr int CW = CL / 2;              // channel pairs (dwords of bf16 / pairs of int8 codes) per lane
  __shared__ __align__(16) float mrg[(2 + D) * kWaves * kMaxGroup];  // the four waves' (m, l, acc) for the merge
  __shared__ int bids[kMaxSplitBlocks];
  __shared__ int last_flag;

  const WorkItem w = work_item(a);
  const int sp = w.sp, h = w.h, s = w.s;
  const int start = w.start;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  auto chan = [&](int j, int i) { return 4 * CH * j + CH * q4 + i; };

  int ids[kIdsPerThread];
  const int nb_spec = fetch_split_ids(a, s, start, w.end, ids);
  // The query group over this lane's channels: fp32 (DOT 0), bf16 pairs (DOT 1, bf16 pool) or fp16 pairs (DOT 1,
  // int8 pool; exact over fp16's normal range).
  float qf[DOT ? 1 : G][DOT ? 1 : CL];
  uint32_t qp[DOT ? G : 1][DOT ? CW : 1];
  float qsum[G];  // MODE 1: the lane's part of the channel sum of q (removes the code bias from the score)
  {
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)s * a.q_ss;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      qsum[g] = 0.f;
      const uint16_t* qg = qrow + (int64_t)(h * G + g) * a.q_sh;
#pragma unroll
      for (int j = 0; j < KC; ++j)
#pragma unroll
        for (int c8 = 0; c8 < CH / 8; ++c8) {
          const u32x4 u = *(const u32x4*)(qg + chan(j, 8 * c8));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = __uint_as_float(u[e] << 16), hi = __uint_as_float(u[e] & 0xffff0000u);
            const int ci = j * CH + 8 * c8 + 2 * e;  // this lane's channel index
            if (MODE == 1) qsum[g] += lo + hi;
            if constexpr (DOT == 0) {
              qf[g][ci] = lo;
              qf[g][ci + 1] = hi;
            } else if constexpr (MODE == 0) {
              qp[g][ci / 2] = u[e];
            } else {
              qp[g][ci / 2] = __builtin_bit_cast(uint32_t, half2_t{(_Float16)lo, (_Float16)hi});
            }
          }
        }
    }
  }
  const int ctx = context_len(a, s);
  if (w.nvalid < 0 && start >= ctx) return;  // grid: a split past this sequence's end
  const int end = max(start, min(w.end, ctx));
  const int nvalid = w.nvalid < 0 ? splits_holding(ctx, a.chunk, a.chunk_old, a.n_old) : w.nvalid;
  commit_split_ids(nb_spec, ids, bids, a.nb);
  __syncthreads();  // block ids staged

  const int esz = MODE == 0 ? 2 : 1;  // bytes per pool element
  const char* kh = (const char*)a.k + (int64_t)h * a.kv_sh * esz;
  const char* vh = (const char*)a.v + (int64_t)h * a.kv_sh * esz;
  const uint16_t* ksh = (const uint16_t*)a.ks + (int64_t)h * a.ks_sh;
  const uint16_t* vsh = (const uint16_t*)a.vs + (int64_t)h * a.vs_sh;
  const int ntile = (end - start + 31) >> 5;
  const int mine = ntile > wave ? (ntile - wave + kWaves - 1) / kWaves : 0;  // tiles wave, wave + 4, ...
  auto tile_t0 = [&](int k) { return start + 32 * (wave + kWaves * k); };
  // Branch-free, as in the MFMA kernels: a second block past the split's end re-reads the first.
  auto load_tile = [&](int k, ValuTile<D, MODE>& tl) {
    const int t0 = tile_t0(k);
    const int bi = (t0 - start) >> 4;
    const int b0 = bids[bi];
    const int b1 = (t0 + 16 < end) ? bids[bi + 1] : b0;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int64_t blk = mt ? b1 : b0;
      const char* kb = kh + blk * a.kv_sn * esz + (int64_t)r * D * esz;
      const char* vb = vh + blk * a.kv_sn * esz + (int64_t)r * D * esz;
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        tl.k[mt][j] = __builtin_nontemporal_load((const u32x4*)(kb + chan(j, 0) * esz));
        tl.v[mt][j] = __builtin_nontemporal_load((const u32x4*)(vb + chan(j, 0) * esz));
      }
      if (MODE == 1) {
        tl.ks[mt] = ksh[blk * a.ks_sn + r];
        tl.vs[mt] = vsh[blk * a.vs_sn + r];
      }
    }
  };

  float m_run[G], l_run[G], bias_w[G];  // bias_w (MODE 1): sum of the p' weights, for the V code bias
  float acc[G][CL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = kNegInf;
    l_run[g] = 0.f;
    bias_w[g] = 0.f;
#pragma unroll
    for (int c = 0; c < CL; ++c) acc[g][c] = 0.f;
  }
  if (MODE == 1) {  // the channel sums of q over all D channels (every lane of a row holds them)
#pragma unroll
    for (int g = 0; g < G; ++g) qsum[g] = sum_over_rows_swap(qsum[g]);
  }
  // INT8 codes are read as 1024 + 128 + c (fp16 via the exponent byte) in the DOT path, as 128 + c (fp32 via the
  // unsigned byte conversions) in the FMA path.
  constexpr float kCodeBias = DOT ? 1152.f : 128.f;

  constexpr float kRescaleSlack = MODE == 0 ? 8.f : 4.f;  // as the MFMA kernels (p' stays in fp16 range)
  auto process_tile = [&](int t0, ValuTile<D, MODE>& tl) {
    float sc[2][G];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int g = 0; g < G; ++g) sc[mt][g] = 0.f;
#pragma unroll
      for (int j = 0; j < KC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t kw = tl.k[mt][j][e];
          if constexpr (MODE == 0) {  // two bf16 channels
            const int cw = (j * CH) / 2 + e;
            if constexpr (DOT) {
#pragma unroll
              for (int g = 0; g < G; ++g)
                sc[mt][g] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, kw),
                                                            __builtin_bit_cast(bf162_t, qp[g][cw]), sc[mt][g], false);
            } else {
              const float k0 = __uint_as_float(kw << 16), k1 = __uint_as_float(kw & 0xffff0000u);
#pragma unroll
              for (int g = 0; g < G; ++g) sc[mt][g] = fmaf(qf[g][2 * cw + 1], k1, fmaf(qf[g][2 * cw], k0, sc[mt][g]));
            }
          } else {  // four int8 channels: codes biased to 128 + c
            const uint32_t u = kw ^ 0x80808080u;
            const int c0 = j * CH + 4 * e;
            if constexpr (DOT) {
              const half2_t lo = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
              const half2_t hi = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
#pragma unroll
              for (int g = 0; g < G; ++g) {
                float x = __builtin_amdgcn_fdot2(lo, __builtin_bit_cast(half2_t, qp[g][c0 / 2]), sc[mt][g], false);
                sc[mt][g] = __builtin_amdgcn_fdot2(hi, __builtin_bit_cast(half2_t, qp[g][c0 / 2 + 1]), x, false);
              }
            } else {
              const float k0 = ubyte_f32(u, 0), k1 = ubyte_f32(u, 1);
              const float k2 = ubyte_f32(u, 2), k3 = ubyte_f32(u, 3);
#pragma unroll
              for (int g = 0; g < G; ++g)
                sc[mt][g] = fmaf(qf[g][c0 + 3], k3, fmaf(qf[g][c0 + 2], k2,
                            fmaf(qf[g][c0 + 1], k1, fmaf(qf[g][c0], k0, sc[mt][g]))));
            }
          }
        }
    }
    const bool partial = t0 + 32 > end;  // wave-uniform
    float mx[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        float x = sum_over_rows_swap(sc[mt][g]);  // over the four q4 lanes: the whole score of token r
        if (MODE == 1) x = (x - kCodeBias * qsum[g]) * f16_bits_to_f32(tl.ks[mt] & 0xffffu);
        if (partial && t0 + 16 * mt + r >= end) x = kNegInf;
        sc[mt][g] = x;
      }
      mx[g] = row16_reduce<true>(fmaxf(sc[0][g], sc[1][g])) * a.scale_log2;
    }
    bool raise = false;
#pragma unroll
    for (int g = 0; g < G; ++g) raise |= mx[g] > m_run[g] + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(raise)) {  // wave-uniform: every lane holds the same maxima
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float m_new = fmaxf(m_run[g], mx[g]);
        const float alpha = fast_exp2(m_run[g] - m_new);
        l_run[g] *= alpha;
        bias_w[g] *= alpha;
#pragma unroll
        for (int c = 0; c < CL; ++c) acc[g][c] *= alpha;
        m_run[g] = m_new;
      }
    }
    float p[2][G];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const float vscale = MODE == 1 ? f16_bits_to_f32(tl.vs[mt] & 0xffffu) : 1.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pp = fast_exp2(fmaf(sc[mt][g], a.scale_log2, -m_run[g]));
        l_run[g] += pp;  // the unscaled p, as the reference keeps l
        p[mt][g] = pp * vscale;
      }
    }
    if (MODE == 0 && partial) {  // bf16 V rows past the end are zeroed: 0-weight garbage must not give NaN
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        if (t0 + 16 * mt + r >= end)
#pragma unroll
          for (int j = 0; j < KC; ++j) tl.v[mt][j] = u32x4{0, 0, 0, 0};
    }
    if constexpr (DOT) {
      uint32_t pw[G];  // (p of token r, p of token 16 + r) as a bf16 (MODE 0) or fp16 (MODE 1) pair
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (MODE == 0)
          pw[g] = __builtin_bit_cast(uint32_t, bf162_t{(__bf16)p[0][g], (__bf16)p[1][g]});
        else
          pw[g] = __builtin_bit_cast(uint32_t, half2_t{(_Float16)p[0][g], (_Float16)p[1][g]});
        if (MODE == 1) {  // the weights the bias of the rounded p' multiplies
          const half2_t ph = __builtin_bit_cast(half2_t, pw[g]);
          bias_w[g] += (float)ph[0] + (float)ph[1];
        }
      }
#pragma unroll
      for (int j = 0; j < KC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w0 = tl.v[0][j][e], w1 = tl.v[1][j][e];
          if constexpr (MODE == 0) {  // channels (2 e, 2 e + 1) of the chunk: pairs over the two tokens
            const int c = j * CH + 2 * e;
            const bf162_t v_lo = __builtin_bit_cast(bf162_t, __builtin_amdgcn_perm(w1, w0, 0x05040100u));
            const bf162_t v_hi = __builtin_bit_cast(bf162_t, __builtin_amdgcn_perm(w1, w0, 0x07060302u));
#pragma unroll
            for (int g = 0; g < G; ++g) {
              acc[g][c] = __builtin_amdgcn_fdot2_f32_bf16(v_lo, __builtin_bit_cast(bf162_t, pw[g]), acc[g][c], false);
              acc[g][c + 1] =
                  __builtin_amdgcn_fdot2_f32_bf16(v_hi, __builtin_bit_cast(bf162_t, pw[g]), acc[g][c + 1], false);
            }
          } else {  // channels 4 e .. 4 e + 3 of the chunk
            const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
            const int c = j * CH + 4 * e;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
              const half2_t vv = bytes_to_f16_pair(u0, u1, kk);
#pragma unroll
              for (int g = 0; g < G; ++g)
                acc[g][c + kk] = __builtin_amdgcn_fdot2(vv, __builtin_bit_cast(half2_t, pw[g]), acc[g][c + kk], false);
            }
          }
        }
    } else {
      if (MODE == 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) bias_w[g] += p[0][g] + p[1][g];
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t vw = tl.v[mt][j][e];
            if constexpr (MODE == 0) {
              const int c = j * CH + 2 * e;
              const float v0 = __uint_as_float(vw << 16), v1 = __uint_as_float(vw & 0xffff0000u);
#pragma unroll
              for (int g = 0; g < G; ++g) {
                acc[g][c] = fmaf(p[mt][g], v0, acc[g][c]);
                acc[g][c + 1] = fmaf(p[mt][g], v1, acc[g][c + 1]);
              }
            } else {
              const uint32_t u = vw ^ 0x80808080u;
              const int c = j * CH + 4 * e;
              const float v0 = ubyte_f32(u, 0), v1 = ubyte_f32(u, 1);
              const float v2 = ubyte_f32(u, 2), v3 = ubyte_f32(u, 3);
#pragma unroll
              for (int g = 0; g < G; ++g) {
                acc[g][c] = fmaf(p[mt][g], v0, acc[g][c]);
                acc[g][c + 1] = fmaf(p[mt][g], v1, acc[g][c + 1]);
                acc[g][c + 2] = fmaf(p[mt][g], v2, acc[g][c + 2]);
                acc[g][c + 3] = fmaf(p[mt][g], v3, acc[g][c + 3]);
              }
            }
          }
    }
  };

  ValuTile<D, MODE> ring[NB];
  if (mine >= 2 * NB) {
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
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      process_tile(tile_t0(k0 + j), ring[j]);
      if (k0 + j + NB < mine) load_tile(k0 + j + NB, ring[j]);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (k0 + NB + j < mine) process_tile(tile_t0(k0 + NB + j), ring[j]);
  } else {
    for (int k = 0; k < mine; ++k) {
      load_tile(k, ring[0]);
      process_tile(tile_t0(k), ring[0]);
    }
  }

  // Each lane's sums cover its tokens r and 16 + r of every tile: sum over the 16 lanes r, remove the INT8 code bias,
  // and hand the wave's state (m, l, acc) to the four-wave merge in LDS.
  float* ms = mrg;
  float* ls = ms + kWaves * kMaxGroup;
  float* accs = ls + kWaves * kMaxGroup;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float lg = row16_reduce<false>(l_run[g]);
    const float bw = MODE == 1 ? row16_reduce<false>(bias_w[g]) : 0.f;
#pragma unroll
    for (int c = 0; c < CL; ++c) {
      float x = row16_reduce<false>(acc[g][c]);
      if (MODE == 1) x -= kCodeBias * bw;
      acc[g][c] = x;
    }
    if (lane == 0) {
      ms[wave * kMaxGroup + g] = m_run[g];
      ls[wave * kMaxGroup + g] = lg;
    }
  }
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < KC; ++j)
#pragma unroll
        for (int i = 0; i < CH; ++i) accs[(wave * kMaxGroup + g) * D + chan(j, i)] = acc[g][j * CH + i];
  }
  __syncthreads();
  finish_split<D, false>(a, s, h, sp, nvalid, ms, ls, accs, &last_flag);
}

template <int D, int MODE, int DOT>
static int launch_g(int G, int nb, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, st, a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? SIPA_OK : fail(SIPA_EHIP, "VALU stream launch failed: %s", hipGetErrorString(e));
  };
  (void)nb;
  constexpr int NB = D == 64 ? 2 : 1;  // head_dim 128: the query and accumulators leave room for one tile in flight
  switch (G) {
    case 6: return go(decode_valu_stream<D, MODE, DOT, 6, NB>);
    case 7: return go(decode_valu_stream<D, MODE, DOT, 7, NB>);
    default: return go(decode_valu_stream<D, MODE, DOT, 8, NB>);
  }
}

bool valu_stream_supported(int D, int G, int mode, int dot) {
  return (D == 64 || D == 128) && (G == 6 || G == 7 || G == 8) && (mode == 0 || mode == 1) && (dot == 0 || dot == 1);
}

int launch_valu_stream(int D, int G, int mode, int dot, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  if (D == 64) {
    if (mode == 0) return dot ? launch_g<64, 0, 1>(G, 2, grid, a, st) : launch_g<64, 0, 0>(G, 2, grid, a, st);
    return dot ? launch_g<64, 1, 1>(G, 2, grid, a, st) : launch_g<64, 1, 0>(G, 2, grid, a, st);
  }
  if (mode == 0) return dot ? launch_g<128, 0, 1>(G, 2, grid, a, st) : launch_g<128, 0, 0>(G, 2, grid, a, st);
  return dot ? launch_g<128, 1, 1>(G, 2, grid, a, st) : launch_g<128, 1, 0>(G, 2, grid, a, st);
}

}  // namespace sipa
