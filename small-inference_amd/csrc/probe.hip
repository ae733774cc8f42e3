// Measurement kernels for bench.py, built into their own library (libsmallinf_probe.so) so that the product's
// C ABI stays the decode path's boundary:
//   sipa_probe_read: a read-only stream of a buffer (contiguous range per workgroup, 16-byte loads, 4..16 in
//                    flight per lane), the measured HBM read ceiling the decode kernel is compared with;
//   sipa_probe_copy: a plain device-to-device copy of a known number of bytes, the reference point that rocprof's
//                    FETCH_SIZE / WRITE_SIZE counters are calibrated against;
//   sipa_probe_paged_read: the HBM reads of one paged-decode call (same grid, block-table staging and load ring as
//                    the decode kernels) without their arithmetic or split merge: the floor of that access pattern.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Each workgroup streams one contiguous range of the buffer (ranges of equal size, in workgroup order), U
// 16-byte loads in flight per lane; NT selects nontemporal loads.
template <int U, bool NT>
__global__ void __launch_bounds__(256) probe_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t lo = (int64_t)blockIdx.x * per;
  const int64_t hi = lo + per < n16 ? lo + per : n16;
  uint32_t acc = 0;
  int64_t i = lo + threadIdx.x;
  for (; i + (U - 1) * 256 < hi; i += U * 256) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * 256) : src[i + u * 256];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < hi; i += 256) {
    const u32x4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;  // keeps the loads live; practically never stores
}

__global__ void __launch_bounds__(256) probe_copy_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                          int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

template <bool NT>
static void launch_read(int unroll, dim3 grid, hipStream_t st, const u32x4* p, int64_t n16, uint32_t* sink) {
  switch (unroll) {
    case 4: hipLaunchKernelGGL((probe_read_kernel<4, NT>), grid, dim3(256), 0, st, p, n16, sink); break;
    case 8: hipLaunchKernelGGL((probe_read_kernel<8, NT>), grid, dim3(256), 0, st, p, n16, sink); break;
    default: hipLaunchKernelGGL((probe_read_kernel<16, NT>), grid, dim3(256), 0, st, p, n16, sink); break;
  }
}

// unroll: 16-byte loads in flight per lane (4, 8 or 16); nontemporal: 1 for nontemporal loads.
extern "C" int32_t sipa_probe_read(const void* src, int64_t bytes, void* sink, int32_t workgroups, int32_t unroll,
                                   int32_t nontemporal, void* stream) {
  if (!src || !sink || bytes < 16 || ((uintptr_t)src & 15) || workgroups <= 0) return -1;
  if (unroll != 4 && unroll != 8 && unroll != 16) return -1;
  hipStream_t st = (hipStream_t)stream;
  if (nontemporal)
    launch_read<true>(unroll, dim3(workgroups), st, (const u32x4*)src, bytes / 16, (uint32_t*)sink);
  else
    launch_read<false>(unroll, dim3(workgroups), st, (const u32x4*)src, bytes / 16, (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int32_t sipa_probe_copy(void* dst, const void* src, int64_t bytes, int32_t workgroups, void* stream) {
  if (!src || !dst || bytes < 16 || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || workgroups <= 0) return -1;
  hipLaunchKernelGGL(probe_copy_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream, (uint4*)dst,
                     (const uint4*)src, bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// sipa_probe_paged_read: the HBM reads of one paged-decode call and nothing else, the floor a decode kernel of this
// layout can reach. Workgroup L takes the token range the decode kernels give it: item L of a work list (items, 8
// int32 each: sequence, KV head, split, splits, start, end), or split sp = L / (S Hkv) of pair L % (S Hkv) on the
// grid, the first n_old splits chunk_old tokens long and the others chunk (every sequence has ctx tokens). 4 waves
// stage the range's block ids in LDS, then each wave streams its 32-token tiles (blocks 2t, 2t + 1 of the range) of
// K and V, row_bytes per token row, 16-byte nontemporal loads, two tiles in flight, like the decode kernels. With
// scale pools (ks and/or vs non-NULL), the range's scale rows of every block are read first (ks_row / vs_row bytes
// each: 32 for per-token scales, D x 2 for per-channel K scales). The data is folded into a word that is never
// stored in practice, so the loads stay live.
namespace {
constexpr int kProbeWaves = 4;
constexpr int kProbeMaxBlocks = 2048;

struct ProbeArgs {
  const uint8_t* k;
  const uint8_t* v;
  const uint8_t* ks;
  const uint8_t* vs;
  const int32_t* bt;
  const int32_t* items;
  int64_t bt_ss, kv_sh, kv_sn, ks_sh, ks_sn, vs_sh, vs_sn;
  int32_t S, Hkv, ctx, chunk, chunk_old, n_old, row_bytes, ks_row, vs_row;
  uint32_t zero;
  uint32_t* sink;
};

__global__ void __launch_bounds__(256) probe_paged_read_kernel(const ProbeArgs a) {
  __shared__ int bids[kProbeMaxBlocks];
  __shared__ u32x4 stage[kProbeWaves * 8 * 64];
  const int L = blockIdx.x;
  int s, h, start, end;
  if (a.items != nullptr) {
    const int32_t* it = a.items + 8 * (int64_t)L;
    s = it[0], h = it[1], start = it[4], end = min(it[5], start + kProbeMaxBlocks * 16);
  } else {
    s = L % a.S, h = (L / a.S) % a.Hkv;
    const int sp = L / (a.S * a.Hkv);
    start = sp <= a.n_old ? sp * a.chunk_old : a.n_old * a.chunk_old + (sp - a.n_old) * a.chunk;
    end = min(start + (sp < a.n_old ? a.chunk_old : a.chunk), a.ctx);
  }
  const int nblk = max((end - start + 15) >> 4, 0);
  for (int j = threadIdx.x; j < nblk; j += 256) bids[j] = a.bt[(int64_t)s * a.bt_ss + (start >> 4) + j];
  __syncthreads();
  uint32_t acc = 0;
  // the range's scale rows, 16 bytes a lane
  for (int arr = 0; arr < 2; ++arr) {
    const uint8_t* base = arr ? a.vs : a.ks;
    if (base == nullptr) continue;
    const int per = (arr ? a.vs_row : a.ks_row) >> 4;
    const int64_t sh = arr ? a.vs_sh : a.ks_sh, sn = arr ? a.vs_sn : a.ks_sn;
    for (int c = threadIdx.x; c < per * nblk; c += 256) {
      const u32x4 x = *(const u32x4*)(base + (int64_t)h * sh + (int64_t)bids[c / per] * sn + 16 * (c % per));
      acc ^= x.x ^ x.w;
    }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ntile = (nblk + 1) >> 1;
  const int mine = ntile > wave ? (ntile - wave + kProbeWaves - 1) / kProbeWaves : 0;  // tiles wave, wave + 4, ...
  const int per_lane = 16 * a.row_bytes / (64 * 16);  // 16-byte loads per lane per block: 2 (2 KiB) or 1 (1 KiB)
  // One tile: blocks 2t, 2t + 1 of K and V, two 16-byte loads per lane and block (a 1 KiB block reads its first
  // kilobyte twice); branch-free. Each ring slot folds into its own word, and a slot's refill address takes that
  // word (& zero, 0 at run time), and a wave-scope fence separates the refill from the other slot's fold: the
  // compiler then waits for one slot at a time and keeps the other one in flight, as in the decode kernels.
  auto load = [&](int kk, u32x4 (&r)[8], uint32_t dep) {
    const int t = wave + kProbeWaves * kk;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int64_t base = (int64_t)h * a.kv_sh + (int64_t)bids[min(2 * t + mt, nblk - 1)] * a.kv_sn + (dep & a.zero);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t o = base + 16 * (lane + 64 * (i < per_lane ? i : 0));
        r[4 * mt + 2 * i] = __builtin_nontemporal_load((const u32x4*)(a.k + o));
        r[4 * mt + 2 * i + 1] = __builtin_nontemporal_load((const u32x4*)(a.v + o));
      }
    }
  };
  // A tile is consumed by LDS stores (the wave's 8 KiB area), as the decode kernels stage their V tiles: the
  // wave-scope fences between a slot's refill and the other slot's stores then keep the compiler from waiting for
  // both slots at once.
  auto fold = [&](const u32x4 (&r)[8], uint32_t& w) {
#pragma unroll
    for (int i = 0; i < 8; ++i) stage[(wave * 8 + i) * 64 + lane] = r[i];
    w ^= 1;
  };
  // a wave-scope fence and barrier: the scheduler keeps each slot's fold after the other slot's refill
  auto order = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  uint32_t a0 = 0, a1 = 0;
  u32x4 r0[8], r1[8];
  if (mine >= 4) {
    load(0, r0, a0);
    load(1, r1, a1);
    int k0 = 0;
    for (; k0 + 4 <= mine; k0 += 2) {
      fold(r0, a0);
      load(k0 + 2, r0, a0);
      order();
      fold(r1, a1);
      load(k0 + 3, r1, a1);
      order();
    }
    // tiles k0, k0 + 1 are loaded; one more may remain
    fold(r0, a0);
    if (k0 + 2 < mine) load(k0 + 2, r0, a0);
    order();
    fold(r1, a1);
    order();
    if (k0 + 2 < mine) fold(r0, a0);
  } else {
    // Every fold overwrites the same LDS words: without the fence between two folds the compiler drops the first
    // one's stores as dead, and that tile's loads with them.
    for (int kk = 0; kk < mine; ++kk) {
      load(kk, r0, a0);
      fold(r0, a0);
      order();
    }
  }
  order();
  acc ^= a0 ^ a1 ^ stage[(wave * 8 + (lane & 7)) * 64 + lane].y;
  if (acc == 0x9e3779b9u) a.sink[L] = acc;
}
}  // namespace

// k, v: pools (row_bytes per token row, 16-token blocks, kv_sh / kv_sn in bytes); bt: [S, ...] block ids with row
// stride bt_ss. Grid (items NULL): every sequence has ctx tokens, split as above (chunk, chunk_old multiples of 32;
// n_old 0 for equal splits). Work list (items non-NULL, n_items entries): each item's range as given. ks, vs: scale
// pools or NULL (rows of ks_row / vs_row bytes, multiples of 16; strides in bytes). Returns 0, or -1 on bad
// arguments.
extern "C" int32_t sipa_probe_paged_read(const void* k, const void* v, const void* ks, const void* vs,
                                         const int32_t* bt, int64_t bt_ss, int32_t S, int32_t Hkv, int32_t ctx,
                                         int32_t chunk, int32_t chunk_old, int32_t n_old, const int32_t* items,
                                         int32_t n_items, int64_t kv_sh, int64_t kv_sn, int64_t ks_sh, int64_t ks_sn,
                                         int32_t ks_row, int64_t vs_sh, int64_t vs_sn, int32_t vs_row,
                                         int32_t row_bytes, void* sink, void* stream) {
  if (!k || !v || !bt || !sink || S <= 0 || Hkv <= 0) return -1;
  if ((row_bytes != 64 && row_bytes != 128) || ((uintptr_t)k & 15) || ((uintptr_t)v & 15) || kv_sh % 16 ||
      kv_sn % 16)
    return -1;
  if ((ks && (ks_row <= 0 || ks_row % 16 || ks_sh % 16 || ks_sn % 16)) ||
      (vs && (vs_row <= 0 || vs_row % 16 || vs_sh % 16 || vs_sn % 16)))
    return -1;
  int64_t wgs;
  if (items) {
    if (n_items <= 0) return -1;
    wgs = n_items;
  } else {
    if (ctx <= 0 || chunk <= 0 || chunk % 32 || chunk / 16 > kProbeMaxBlocks || n_old < 0 ||
        (n_old > 0 && (chunk_old <= 0 || chunk_old % 32 || chunk_old / 16 > kProbeMaxBlocks)))
      return -1;
    const int64_t covered = (int64_t)n_old * chunk_old;
    const int64_t splits = covered >= ctx ? (ctx + chunk_old - 1) / chunk_old : n_old + (ctx - covered + chunk - 1) / chunk;
    wgs = (int64_t)S * Hkv * splits;
  }
  ProbeArgs a{(const uint8_t*)k, (const uint8_t*)v, (const uint8_t*)ks, (const uint8_t*)vs, bt, items, bt_ss, kv_sh,
              kv_sn, ks_sh, ks_sn, vs_sh, vs_sn, S, Hkv, ctx, chunk, chunk_old, n_old, row_bytes, ks_row, vs_row, 0u,
              (uint32_t*)sink};
  hipLaunchKernelGGL(probe_paged_read_kernel, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
