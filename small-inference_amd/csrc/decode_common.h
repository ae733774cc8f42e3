// Device code shared by the decode kernels (decode.hip: bf16 MFMA, VALU, combine; decode_int8.hip: INT8 MFMA):
// grid-to-work mapping, the split merge (LDS merge of the waves, coherent partials, last-arriving combine), and
// the MFMA kernels' common prologue and epilogue.
#pragma once

#include "sipa_common.h"

namespace sipa {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr int kMaxSplitBlocks = 2048;  // block ids of one split the MFMA kernel stages in LDS (32768 tokens)

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The larger of two scores as gfx950's v_maximum(3)_f32. fmaxf lowers, in the IEEE mode kernels run in, to
// v_max_f32 with every operand first quieted by a v_max_f32 x, x of its own; maximum needs no quieting and fuses
// three operands. It differs from fmaxf only where a score max never goes: a NaN operand (propagated rather than
// dropped) and -0 against +0 (+0 wins).
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the lanes of an MFMA accumulator column).
__device__ __forceinline__ float max_over_rows(float x) {
  x = vmax(x, __shfl_xor(x, 16));
  return vmax(x, __shfl_xor(x, 32));
}

__device__ __forceinline__ float sum_over_rows(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// The same reductions with gfx950's row-swap permutes: permlane16_swap(x, x) yields the even and the odd 16-lane
// row of each row pair, permlane32_swap(x, x) the low and the high half-wave, so each step is one permute and one
// VALU op with no LDS round trip; every lane combines the same two operands in the same order, so all four lanes
// get the same bits. Measured: 3-6% faster in the prefill kernel, but the decode kernels ran slower with them
// (the ragged split-grid case 52 -> 65 us), so only the prefill kernel uses these.
__device__ __forceinline__ float max_over_rows_swap(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float sum_over_rows_swap(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Token ranges of the split grid: the first n_old splits of every sequence hold chunk_old tokens, the others chunk
// (n_old = 0: all chunk). On a grid of two workgroups per CU the first CU-count workgroups (the earlier-dispatched
// of each CU's pair) are given the longer splits: the older workgroup of a CU wins the instruction-issue arbitration
// and streams faster while both run, so with equal splits it finished ~5 us before its partner, which then ran
// alone at half the CU's occupancy.
__device__ __forceinline__ int split_begin(int sp, int chunk, int chunk_old, int n_old) {
  return sp <= n_old ? sp * chunk_old : n_old * chunk_old + (sp - n_old) * chunk;
}

__device__ __forceinline__ int split_length(int sp, int chunk, int chunk_old, int n_old) {
  return sp < n_old ? chunk_old : chunk;
}

// Splits that hold tokens of a ctx-token sequence.
__device__ __forceinline__ int splits_holding(int ctx, int chunk, int chunk_old, int n_old) {
  const int b = n_old * chunk_old;
  return ctx <= b ? (ctx + chunk_old - 1) / chunk_old : n_old + (ctx - b + chunk - 1) / chunk;
}

// Without a work list the grid is one-dimensional, sequence index fastest, then KV head, then split. The hardware
// hands workgroup L to XCD L % 8, so consecutive sequences land on different XCDs and a ragged batch's work spreads
// evenly over them; and every sequence's first split (the only one a short sequence has) is dispatched before any
// second one. With a work list, workgroup L takes item L: {sequence, KV head, split, splits of that pair, start,
// end}. Item fields are clamped into range, so a list that does not match the context lengths gives wrong
// results but no out-of-bounds access.
struct WorkItem {
  int s, h, sp;
  int start, end;  // tokens [start, end) before clamping to the context length
  int nvalid;      // splits of (s, h) that hold tokens (work list); -1: derived from the context length
};

__device__ __forceinline__ WorkItem work_item(const DecodeArgs& a) {
  const int L = blockIdx.x;
  if (a.items != nullptr) {
    const int4* it = (const int4*)(a.items + 8 * (int64_t)L);
    const int4 x = it[0], y = it[1];
    WorkItem w;
    w.s = min(max(x.x, 0), a.S - 1);
    w.h = min(max(x.y, 0), a.Hkv - 1);
    w.sp = min(max(x.z, 0), a.splits - 1);
    w.nvalid = min(max(x.w, 1), a.splits);
    w.start = min(max(y.x, 0), a.max_ctx);
    w.end = min(max(y.y, w.start), min(a.max_ctx, w.start + kMaxSplitBlocks * 16));
    return w;
  }
  const int sh = L % (a.S * a.Hkv);
  const int sp = L / (a.S * a.Hkv);
  const int b = split_begin(sp, a.chunk, a.chunk_old, a.n_old);
  return WorkItem{sh % a.S, sh / a.S, sp, b, min(b + split_length(sp, a.chunk, a.chunk_old, a.n_old), a.max_ctx), -1};
}

// The fields a bf16 decode workgroup needs before its first K/V load, passed as leading scalar kernel arguments
// that gfx950 preloads into SGPRs at wave launch (-amdgpu-kernarg-preload-count): the block-table and context-length
// loads then start without waiting for the kernel-argument fetch (a memory round trip of about 0.5 us).
struct HotArgs {
  const int32_t* bt;     // block tables
  const int32_t* ctx;    // context lengths
  const int32_t* items;  // work list or NULL
  int32_t bt_ss;         // block-table row stride (elements)
  int32_t SH;            // sequences x KV heads
  int32_t S, chunk, max_ctx, bt_w;  // equal splits of chunk tokens (the host gives the bf16 kernel no two-class grid)
};

__device__ __forceinline__ WorkItem work_item(const HotArgs& hp, const DecodeArgs& a) {
  const int L = blockIdx.x;
  if (hp.items != nullptr) {
    const int4* it = (const int4*)(hp.items + 8 * (int64_t)L);
    const int4 x = it[0], y = it[1];
    WorkItem w;
    w.s = min(max(x.x, 0), hp.S - 1);
    w.h = min(max(x.y, 0), hp.SH / hp.S - 1);
    w.sp = min(max(x.z, 0), a.splits - 1);
    w.nvalid = min(max(x.w, 1), a.splits);
    w.start = min(max(y.x, 0), hp.max_ctx);
    w.end = min(max(y.y, w.start), min(hp.max_ctx, w.start + kMaxSplitBlocks * 16));
    return w;
  }
  const int sh = L % hp.SH;
  const int sp = L / hp.SH;
  return WorkItem{sh % hp.S, sh / hp.S, sp, sp * hp.chunk, min(sp * hp.chunk + hp.chunk, hp.max_ctx), -1};
}

template <bool OUT_F32>
__device__ __forceinline__ void store_out(const DecodeArgs& a, int s, int hq, int d, float v) {
  const int64_t i = (int64_t)s * a.o_ss + (int64_t)hq * a.o_sh + d;
  if (OUT_F32)
    ((float*)a.out)[i] = v;
  else
    ((uint16_t*)a.out)[i] = f32_to_bf16_bits(v);
}

// Partials that another workgroup of the same launch merges are written and read with agent-scope accesses:
// relaxed agent-scope atomics, which gfx950 executes as global_store / global_load with the sc1 bit, or buffer
// loads and stores with that same bit (partial_rows below); both write through to and read from the point of
// coherence of all XCDs. Ordering then needs only the completion of this workgroup's stores
// (s_waitcnt vmcnt(0)) before its counter increment, not an agent-scope fence, which would write back and
// invalidate the whole L2 of the XCD once per workgroup.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_coherent(float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Four consecutive outputs. A bf16 row piece on a 4-byte boundary goes out as two packed words written through
// to memory (relaxed agent-scope stores, sc1), so the launch ends with no dirty output lines in L2 to release
// (C2: 26.17 -> 26.03 us against four 2-byte write-back stores).
template <bool OUT_F32>
__device__ __forceinline__ void store_out4(const DecodeArgs& a, int s, int hq, int d0, f32x4 v) {
  const int64_t i = (int64_t)s * a.o_ss + (int64_t)hq * a.o_sh + d0;
  if (!OUT_F32) {
    uint16_t* o = (uint16_t*)a.out + i;
    if (((uintptr_t)o & 3) == 0) {
      const uint32_t w0 = pack_bf16x2(v[0], v[1]);
      const uint32_t w1 = pack_bf16x2(v[2], v[3]);
      __hip_atomic_store((uint32_t*)o, w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store((uint32_t*)o + 1, w1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) store_out<OUT_F32>(a, s, hq, d0 + k, v[k]);
}

// The partial rows of one (s, h): [G][splits][D] floats from part + ((s Hq + h G) splits) D, as a raw buffer
// resource (gfx9 descriptor word 3). Loads and stores through it with the sc1 cache-policy bit (aux 16) are
// agent-coherent, like the relaxed agent-scope atomics above, but move 16 bytes per lane in one instruction.
constexpr int kAuxSc1 = 16;
// The sc0 bit alone (aux 1): workgroup-scope loads, served by the XCD's L2 (coherent with every store made on the
// same XCD) once the CU's L1 holds no copy of the line: the merge invalidates the L1 before using them.
constexpr int kAuxSc0 = 1;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rows(const DecodeArgs& a, int s, int h, int D) {
  float* base = a.part + ((int64_t)s * a.Hq + (int64_t)h * a.G) * a.splits * D;
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, a.G * a.splits * D * 4, 0x00020000);
}

// Where a merge reads the split partials from: plainly (the separate combine kernel, a later launch), from the
// merging workgroup's XCD's L2 (every split of the pair ran on that XCD: their write-through stores updated it),
// or through memory with agent-coherent loads (splits on several XCDs).
enum MergeLoads { kMergePlain = 0, kMergeL2 = 1, kMergeMemory = 2 };

// One round of the merge: up to KB splits j0 .. j0 + KB - 1 of row0 (query head g of the pair), every load
// issued before the first is used. Entries past nvalid re-read the last split and get weight 0 (branch-free).
template <int KB, int D, int POL>
__device__ __forceinline__ void combine_round(const DecodeArgs& a, __amdgpu_buffer_rsrc_t rows,
                                              __amdgpu_buffer_rsrc_t mrows, __amdgpu_buffer_rsrc_t lrows,
                                              int64_t row0, int g, int c, int j0, int nvalid, float& M, float& den,
                                              f32x4& num) {
  constexpr int AUX = POL == kMergeL2 ? kAuxSc0 : kAuxSc1;
  float mj[KB], lj[KB];
  f32x4 pj[KB];
#pragma unroll
  for (int u = 0; u < KB; ++u) {
    const int j = min(j0 + u, nvalid - 1);
    if constexpr (POL == kMergePlain) {
      mj[u] = a.pm[row0 + j];
      lj[u] = a.pl[row0 + j];
      pj[u] = *(const f32x4*)(a.part + (row0 + j) * D + 4 * c);
    } else {
      const int e = g * a.splits + j;
      mj[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(mrows, e * 4, 0, AUX));
      lj[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lrows, e * 4, 0, AUX));
      pj[u] = __builtin_amdgcn_raw_buffer_load_b128(rows, (e * D + 4 * c) * 4, 0, AUX);
    }
  }
#pragma unroll
  for (int u = 0; u < KB; ++u)
    if (j0 + u >= nvalid) mj[u] = kNegInf;
  float mb = M;
#pragma unroll
  for (int u = 0; u < KB; ++u) mb = fmaxf(mb, mj[u]);
  const float rescale = fast_exp2(M - mb);  // 0 on the first round (M = -inf)
  den *= rescale;
  num *= rescale;
#pragma unroll
  for (int u = 0; u < KB; ++u) {
    const float w = fast_exp2(mj[u] - mb);  // 0 for the padding entries (m = -inf)
    den += w * lj[u];
    num += w * pj[u];
  }
  M = mb;
}

// Merge the split partials of (s, h) for every query head of the group: rows [h*G, h*G + G). One thread per
// (query head, 4-channel quad), so all loads of a round are in flight together; 4 (nvalid <= 4), 8 (<= 8) or 16
// splits per round, merged online, so up to 8 splits cost one memory round trip and 32 cost two. POL: where the
// partials are read from (MergeLoads).
template <int D, bool OUT_F32, int POL>
__device__ void combine_group(const DecodeArgs& a, int s, int h, int nvalid) {
  constexpr int Q = D / 4;
  const int G = a.G;
  const __amdgpu_buffer_rsrc_t rows = partial_rows(a, s, h, D);
  const int64_t pair0 = ((int64_t)s * a.Hq + (int64_t)h * G) * a.splits;
  const __amdgpu_buffer_rsrc_t mrows = __builtin_amdgcn_make_buffer_rsrc(a.pm + pair0, (short)0, G * a.splits * 4,
                                                                         0x00020000);
  const __amdgpu_buffer_rsrc_t lrows = __builtin_amdgcn_make_buffer_rsrc(a.pl + pair0, (short)0, G * a.splits * 4,
                                                                         0x00020000);
  for (int idx = threadIdx.x; idx < G * Q; idx += kThreads) {
    const int g = idx / Q, c = idx % Q;
    const int64_t row0 = pair0 + (int64_t)g * a.splits;
    float M = kNegInf, den = 0.f;
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    if (nvalid <= 4) {
      combine_round<4, D, POL>(a, rows, mrows, lrows, row0, g, c, 0, nvalid, M, den, num);
    } else if (nvalid <= 8) {
      combine_round<8, D, POL>(a, rows, mrows, lrows, row0, g, c, 0, nvalid, M, den, num);
    } else {
      for (int j0 = 0; j0 < nvalid; j0 += 16)
        combine_round<16, D, POL>(a, rows, mrows, lrows, row0, g, c, j0, nvalid, M, den, num);
    }
    store_out4<OUT_F32>(a, s, h * G + g, 4 * c, num / den);
  }
}

// After this workgroup's partial stores are issued: once they have completed (reached the point of coherence),
// count the partial; the workgroup that brings the count of (s, h) to nvalid merges every partial and resets the
// counter for the next launch. On the (sequence, KV head, split) grid with S Hkv a multiple of 8, every split of
// (s, h) has the same workgroup id mod 8, the XCD the dispatcher deals it to; each workgroup checks that it ran
// there (XCC_ID) and counts +2^16 if not (and always on a work list, whose items go anywhere). The merger reads
// from its L2 when no split of the pair counted away, through memory otherwise.
template <int D, bool OUT_F32>
__device__ void publish_and_merge(const DecodeArgs& a, int s, int h, int nvalid, int* last_flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const bool may_share = a.items == nullptr && (a.S * a.Hkv) % 8 == 0;
    const int away = !may_share || (int)(xcc & 0xf) != (int)(blockIdx.x & 7);
    const int prev = __hip_atomic_fetch_add(a.counters + (int64_t)s * a.Hkv + h, 1 + (away << 16),
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last_flag = (prev & 0xffff) == nvalid - 1 ? 1 + ((prev >> 16) + away == 0) : 0;
  }
  __syncthreads();
  if (!*last_flag) return;
  if (*last_flag == 2) {
    // sc0 loads are workgroup-scope: outside threadgroup-split mode the CU's L1 may serve them. A line of partials
    // this CU read earlier in the launch (another pair's merge, with rows sharing the line) could be stale there,
    // so the L1 is invalidated first; the loads then come from the XCD's L2, which every split's write-through
    // stores passed.
    asm volatile("buffer_inv sc0" ::: "memory");
    combine_group<D, OUT_F32, kMergeL2>(a, s, h, nvalid);
  } else
    combine_group<D, OUT_F32, kMergeMemory>(a, s, h, nvalid);
  if (threadIdx.x == 0)
    __hip_atomic_store(a.counters + (int64_t)s * a.Hkv + h, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge the four waves' states (ms, ls [4][16], accs [4][16][D] in LDS, after a barrier) and write the output
// (whole sequence in this workgroup) or the split partial; with fused merging, the last split workgroup of
// (s, h) to arrive then combines all partials.
template <int D, bool OUT_F32>
__device__ void finish_split(const DecodeArgs& a, int s, int h, int sp, int nvalid, const float* ms,
                             const float* ls, const float* accs, int* last_flag) {
  const int G = a.G;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int g = idx / D, d = idx % D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ms[w * kMaxGroup + g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = ms[w * kMaxGroup + g];
      const float e = (mw == kNegInf) ? 0.f : fast_exp2(mw - M);  // a wave with no tokens drops out
      L += e * ls[w * kMaxGroup + g];
      O += e * accs[(w * kMaxGroup + g) * D + d];
    }
    if (nvalid == 1) {
      store_out<OUT_F32>(a, s, h * G + g, d, O / L);
    } else {
      const int64_t row = ((int64_t)s * a.Hq + h * G + g) * a.splits + sp;
      if (a.fused) {
        store_coherent(a.part + row * D + d, O);
        if (d == 0) {
          store_coherent(a.pm + row, M);
          store_coherent(a.pl + row, L);
        }
      } else {
        a.part[row * D + d] = O;
        if (d == 0) {
          a.pm[row] = M;
          a.pl[row] = L;
        }
      }
    }
  }
  if (nvalid == 1 || !a.fused) return;
  publish_and_merge<D, OUT_F32>(a, s, h, nvalid, last_flag);
}

// ---- MFMA kernels --------------------------------------------------------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// Transposing LDS read (gfx950 ds_read_b64_tr_b16). Within each group of 16 lanes, lane j passes the address of a
// 4-element (8-byte) chunk M[j]; lane i receives M[4 k + i / 4][i % 4], k = 0..3. With lane j of group q4 pointing
// at row 4 q4 + j / 4, columns c0 + 4 (j % 4) .. + 3 of a row-major tile, lane (r, q4) receives rows
// 4 q4 .. 4 q4 + 3 of column c0 + r: the A-operand order of the P.V MFMA.
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p));
}

// Lane (r, q4)'s element offset into a row-major [32][pitch] 16-bit tile for lds_read_tr16: row 4 q4 + r / 4,
// column 4 (r % 4).
__device__ __forceinline__ int tr16_offset(int r, int q4, int pitch) { return (4 * q4 + (r >> 2)) * pitch + 4 * (r & 3); }

// The 8 k-slots of the P.V A operand for columns c0 .. c0 + 15: slot i is row 16 (i / 4) + 4 q4 + i % 4.
template <typename T8>
__device__ __forceinline__ T8 read_v_operand(const uint16_t* tile, int tr_off, int pitch, int c0) {
  const i16x4 lo = lds_read_tr16(tile + tr_off + c0);
  const i16x4 hi = lds_read_tr16(tile + tr_off + 16 * pitch + c0);
  return __builtin_bit_cast(T8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <int D>
struct MfmaSmem {
  static constexpr int kVPitch = D + 8;                                // bf16 elements per LDS row of V
  static constexpr int kVBytes = kWaves * 32 * kVPitch * 2;            // per-wave [32 tok][D] V tiles
  static constexpr int kMergePitch = D + 4;                           // floats per LDS row of a wave's O^T
  static constexpr int kMergeBytes = (2 * kWaves * kMaxGroup + kWaves * kMaxGroup * kMergePitch) * 4;
  static constexpr int kBytes = kVBytes > kMergeBytes ? kVBytes : kMergeBytes;
};

// K/V are streamed once per call: nontemporal loads keep them from displacing anything in the caches.
__device__ __forceinline__ u32x4 stream_load(const uint16_t* p) { return __builtin_nontemporal_load((const u32x4*)p); }

// One 32-token tile (two blocks) of K and V in registers: K in the QK A-operand layout, V as 16-byte row chunks.
template <int D>
struct KVTile {
  u32x4 k[2][D / 32];
  u32x4 v[2][D / 32];
};

// ---- prologue / epilogue shared by the MFMA kernels ----------------------------------------------------------

// Issue the loads of a split's block ids for the longest possible split (every table row covers max_ctx tokens)
// before ctx[s] is known, so that the first K/V loads wait for one memory round trip instead of two.
constexpr int kIdsPerThread = kMaxSplitBlocks / kThreads;

__device__ __forceinline__ int fetch_split_ids(const int32_t* bt, int64_t bt_ss, int bt_w, int s, int start,
                                               int end_spec, int (&ids)[kIdsPerThread]) {
  const int nb_spec = min((end_spec - start + 15) >> 4, bt_w - (start >> 4));  // never past the row's width
  const int32_t* btr = bt + (int64_t)s * bt_ss + (start >> 4);
#pragma unroll
  for (int i = 0; i < kIdsPerThread; ++i) {
    const int j = threadIdx.x + kThreads * i;
    ids[i] = (j < nb_spec) ? btr[j] : 0;
  }
  return nb_spec;
}

// The same without a branch per load: every thread issues all N loads (entries past the split read its last id
// again, an empty split reads column 0 of its row), so no use of one id can be placed between the loads and the
// next memory operations: the ids, the context length and the kernel arguments are then in flight together and
// the first K/V loads wait for one round trip. N x kThreads ids: the longest split the kernel stages.
template <int N>
__device__ __forceinline__ int fetch_split_ids_flat(const int32_t* bt, int64_t bt_ss, int bt_w, int s, int start,
                                                    int end_spec, int (&ids)[N]) {
  const int nb_spec = min((end_spec - start + 15) >> 4, bt_w - (start >> 4));  // never past the row's width
  const int last = max(nb_spec - 1, 0);
  const int32_t* btr = bt + (int64_t)s * bt_ss + (nb_spec > 0 ? (start >> 4) : 0);
#pragma unroll
  for (int i = 0; i < N; ++i) ids[i] = btr[min((int)threadIdx.x + kThreads * i, last)];
  return nb_spec;
}

// Stages every thread's ids (N x kThreads entries of bids, those past the split unused), clamped into the pool,
// without a branch.
template <int N>
__device__ __forceinline__ void commit_split_ids_flat(const int (&ids)[N], int* bids, int nblocks) {
#pragma unroll
  for (int i = 0; i < N; ++i) bids[threadIdx.x + kThreads * i] = min(max(ids[i], 0), nblocks - 1);
}

// Ids outside the pool are clamped into it: a bad table gives wrong results, never an access out of bounds.
__device__ __forceinline__ int fetch_split_ids(const DecodeArgs& a, int s, int start, int end_spec,
                                               int (&ids)[kIdsPerThread]) {
  return fetch_split_ids(a.bt, a.bt_ss, a.bt_w, s, start, end_spec, ids);
}

__device__ __forceinline__ void commit_split_ids(int nb_spec, const int (&ids)[kIdsPerThread], int* bids,
                                                 int nblocks) {
#pragma unroll
  for (int i = 0; i < kIdsPerThread; ++i) {
    const int j = threadIdx.x + kThreads * i;
    if (j < nb_spec) bids[j] = min(max(ids[i], 0), nblocks - 1);
  }
}

// A sequence's context length as the kernels use it: at most max_context, so that the splits a sequence reports
// (and the merge waits for) are always ones the launch has.
__device__ __forceinline__ int context_len(const DecodeArgs& a, int s) { return min(a.ctx[s], a.max_ctx); }

// The staging slot of sequence s's partial last block (INT8 per-channel K): -1 (none) stays -1, slots past the
// staging pool are clamped into it.
__device__ __forceinline__ int tail_slot(const DecodeArgs& a, int s) { return min(a.tail[s], a.n_stage - 1); }

// MFMA epilogue: each wave's softmax state (m_run per lane for head g = r, l_run partial per lane, acc in the
// O^T accumulator layout: lane (r, q4) holds head r, channels 16 dt + 4 q4 + i) goes to LDS; then thread
// (wave, r, q4) merges the four waves for head r and the channel quads 4 wave + q4 + 16 j, with all its LDS reads
// in flight together, and writes the output (whole sequence in this workgroup) or the split partial.
template <int D, bool OUT_F32>
__device__ __forceinline__ void mfma_epilogue(const DecodeArgs& a, int s, int h, int sp, int nvalid, float m_run,
                                              float l_run, const f32x4 (&acc)[D / 16], char* smem,
                                              int* last_flag) {
  constexpr int P = MfmaSmem<D>::kMergePitch;
  constexpr int J = D / 64;  // channel quads per thread
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  l_run = sum_over_rows(l_run);
  __syncthreads();  // every wave is done with its LDS tiles: the LDS becomes the merge buffer
  float2* ml = (float2*)smem;                       // [kWaves][16] (m, l)
  float* accs = (float*)(ml + kWaves * kMaxGroup);  // [kWaves][16][P]
  if (q4 == 0) ml[wave * kMaxGroup + r] = float2{m_run, l_run};
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) *(f32x4*)(accs + (wave * kMaxGroup + r) * P + 16 * dt + 4 * q4) = acc[dt];
  __syncthreads();
  const int G = a.G;
  if (r < G) {
    float2 mw[kWaves];
    f32x4 aw[J][kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mw[w] = ml[w * kMaxGroup + r];
#pragma unroll
      for (int j = 0; j < J; ++j) aw[j][w] = *(const f32x4*)(accs + (w * kMaxGroup + r) * P + 4 * (4 * wave + q4 + 16 * j));
    }
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mw[w].x);
    float L = 0.f;
    f32x4 O[J];
#pragma unroll
    for (int j = 0; j < J; ++j) O[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = (mw[w].x == kNegInf) ? 0.f : fast_exp2(mw[w].x - M);  // a wave with no tokens drops out
      L += e * mw[w].y;
#pragma unroll
      for (int j = 0; j < J; ++j) O[j] += e * aw[j][w];
    }
    const int64_t row = ((int64_t)s * a.Hq + h * G + r) * a.splits + sp;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int d0 = 4 * (4 * wave + q4 + 16 * j);
      if (nvalid == 1) {
        store_out4<OUT_F32>(a, s, h * G + r, d0, O[j] / L);
      } else if (a.fused) {
        __builtin_amdgcn_raw_buffer_store_b128(O[j], partial_rows(a, s, h, D), ((r * a.splits + sp) * D + d0) * 4, 0,
                                               kAuxSc1);
      } else {
        *(f32x4*)(a.part + row * D + d0) = O[j];
      }
    }
    if (nvalid > 1 && wave == 0 && q4 == 0) {
      if (a.fused) {
        store_coherent(a.pm + row, M);
        store_coherent(a.pl + row, L);
      } else {
        a.pm[row] = M;
        a.pl[row] = L;
      }
    }
  }
  if (nvalid == 1 || !a.fused) return;
  publish_and_merge<D, OUT_F32>(a, s, h, nvalid, last_flag);
}

// VALU streaming kernels (decode_valu_stream.hip): bf16 q, 16-token blocks, head_dim 64/128, groups of 6-8, pools
// in bf16 (mode 0) or int8 per token (mode 1); dot = 0: fp32 FMAs, 1: v_dot2 pair products.
bool valu_stream_supported(int D, int G, int mode, int dot);
int launch_valu_stream(int D, int G, int mode, int dot, dim3 grid, const DecodeArgs& a, hipStream_t st);

// INT8 MFMA kernels (decode_int8.hip). mode: 1 per-token K scales, 2 per-(block, channel) K scales,
// 3 per-(head, channel) K scales (mode 2 with a zero block stride). nb: tiles in flight per wave.
int launch_mfma_int8(int D, int mode, int nb, dim3 grid, const DecodeArgs& a, hipStream_t st);

}  // namespace sipa
