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
// layout can reach. Workgroup (sequence s, KV head h, split sp) of a (S, Hkv, splits) grid, 4 waves, stages the
// split's block ids in LDS, then each wave streams its 32-token tiles (blocks 2t, 2t + 1 of the split) of K and V,
// row_bytes per token row, 16-byte nontemporal loads, two tiles in flight, like the decode kernels. With token-scale
// pools (ks, vs: row_bytes 0 when absent), the split's 32-byte scale rows of every block are read first, as the INT8
// kernel stages them. The data is folded into a word that is never stored in practice, so the loads stay live.
namespace {
constexpr int kProbeWaves = 4;
constexpr int kProbeMaxBlocks = 2048;

__global__ void __launch_bounds__(256) probe_paged_read_kernel(const uint8_t* __restrict__ k,
                                                                const uint8_t* __restrict__ v,
                                                                const uint8_t* __restrict__ ks,
                                                                const uint8_t* __restrict__ vs,
                                                                const int32_t* __restrict__ bt, int64_t bt_ss, int S,
                                                                int Hkv, int chunk, int ctx, int64_t kv_sh,
                                                                int64_t kv_sn, int64_t sc_sh, int64_t sc_sn,
                                                                int row_bytes, uint32_t zero,
                                                                uint32_t* __restrict__ sink) {
  __shared__ int bids[kProbeMaxBlocks];
  __shared__ u32x4 stage[kProbeWaves * 8 * 64];
  const int L = blockIdx.x;
  const int s = L % S, h = (L / S) % Hkv, sp = L / (S * Hkv);
  const int start = sp * chunk, end = min(start + chunk, ctx);
  const int nblk = (end - start + 15) >> 4;
  for (int j = threadIdx.x; j < nblk; j += 256) bids[j] = bt[(int64_t)s * bt_ss + (start >> 4) + j];
  __syncthreads();
  uint32_t acc = 0;
  if (ks != nullptr) {  // the split's token scales: 16-byte loads, half a block's 32-byte row each
    for (int c = threadIdx.x; c < 2 * nblk; c += 256) {
      const int64_t off = (int64_t)h * sc_sh + (int64_t)bids[c >> 1] * sc_sn + 16 * (c & 1);
      const u32x4 a = *(const u32x4*)(ks + off), b = *(const u32x4*)(vs + off);
      acc ^= a.x ^ b.w;
    }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ntile = (nblk + 1) >> 1;
  const int mine = ntile > wave ? (ntile - wave + kProbeWaves - 1) / kProbeWaves : 0;  // tiles wave, wave + 4, ...
  const int per_lane = 16 * row_bytes / (64 * 16);  // 16-byte loads per lane per block: 2 (2 KiB) or 1 (1 KiB)
  // One tile: blocks 2t, 2t + 1 of K and V, two 16-byte loads per lane and block (a 1 KiB block reads its first
  // kilobyte twice); branch-free. Each ring slot folds into its own word, and a slot's refill address takes that
  // word (& zero, 0 at run time), and a wave-scope fence separates the refill from the other slot's fold: the
  // compiler then waits for one slot at a time and keeps the other one in flight, as in the decode kernels.
  auto load = [&](int kk, u32x4 (&r)[8], uint32_t dep) {
    const int t = wave + kProbeWaves * kk;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int64_t base = (int64_t)h * kv_sh + (int64_t)bids[min(2 * t + mt, nblk - 1)] * kv_sn + (dep & zero);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t o = base + 16 * (lane + 64 * (i < per_lane ? i : 0));
        r[4 * mt + 2 * i] = __builtin_nontemporal_load((const u32x4*)(k + o));
        r[4 * mt + 2 * i + 1] = __builtin_nontemporal_load((const u32x4*)(v + o));
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
    fold(r1, a1);
    if (k0 + 2 < mine) fold(r0, a0);
  } else {
    for (int kk = 0; kk < mine; ++kk) {
      load(kk, r0, a0);
      fold(r0, a0);
    }
  }
  order();
  acc ^= a0 ^ a1 ^ stage[(wave * 8 + (lane & 7)) * 64 + lane].y;
  if (acc == 0x9e3779b9u) sink[L] = acc;
}
}  // namespace

// k, v: pools (row_bytes per token row, 16-token blocks, kv_sh / kv_sn in bytes); bt: [S, >= ceil(ctx / 16)] block
// ids with row stride bt_ss; every sequence has ctx tokens, cut into splits of `chunk` (a multiple of 32). ks, vs:
// optional token-scale pools (32-byte rows per block, strides in bytes) or NULL. Returns 0, or -1 on bad arguments.
extern "C" int32_t sipa_probe_paged_read(const void* k, const void* v, const void* ks, const void* vs,
                                         const int32_t* bt, int64_t bt_ss, int32_t S, int32_t Hkv, int32_t ctx,
                                         int32_t chunk, int64_t kv_sh, int64_t kv_sn, int64_t sc_sh, int64_t sc_sn,
                                         int32_t row_bytes, void* sink, void* stream) {
  if (!k || !v || !bt || !sink || S <= 0 || Hkv <= 0 || ctx <= 0 || chunk <= 0 || chunk % 32) return -1;
  if (chunk / 16 > kProbeMaxBlocks || (row_bytes != 64 && row_bytes != 128) || ((uintptr_t)k & 15) ||
      ((uintptr_t)v & 15) || kv_sh % 16 || kv_sn % 16 || (ks && (!vs || sc_sh % 16 || sc_sn % 16)))
    return -1;
  const int splits = (ctx + chunk - 1) / chunk;
  hipLaunchKernelGGL(probe_paged_read_kernel, dim3(S * Hkv * splits), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)k, (const uint8_t*)v, (const uint8_t*)ks, (const uint8_t*)vs, bt, bt_ss, S, Hkv,
                     chunk, ctx, kv_sh, kv_sn, sc_sh, sc_sn, row_bytes, 0u, (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
