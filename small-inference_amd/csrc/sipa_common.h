// Shared definitions of the gfx950 paged-attention decode library: vector types, element conversions, the
// kernel argument block, and host-side error reporting.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smallinf_hip.h"

namespace sipa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;          // waves per decode workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxGroup = 16;      // query heads per KV head the kernels accept (the MFMA tile height)
constexpr int kChunkAlign = 64;    // split chunks are multiples of 64 tokens (the reference's TILE)
constexpr int kMinChunk = 256;     // smallest split the CU-count policy makes
constexpr int kMaxChunk = 2048;    // largest split the policy makes when the grid is already full
constexpr int kLatencyChunk = 512;  // smallest split of a small batch past kShortSplits splits
constexpr int kShortChunk = 128;    // smallest split of a short context ...
constexpr int kShortSplits = 8;     // ... cut into at most this many (one merge round)
// Split workspaces (decode and prefill) keep their merge counters in a fixed region at the start, which no call
// writes partials into: every call leaves the counters it used at zero, so one zero-filled workspace serves calls
// of any size, decode and prefill alike, in any order on one stream.
constexpr int64_t kCounterBytes = 1 << 18;
constexpr int kMaxCounters = (int)(kCounterBytes / 4);
constexpr int kMaxInt8Split = 4096;  // longest split of the INT8 MFMA kernels (their token scales are staged in LDS)

// ---- element conversions -------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t u16) { return __uint_as_float(u16 << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);  // round to nearest even (v_cvt_pk_bf16_f32)
}

// Two values rounded to nearest even and packed (lo in bits 0-15), as one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32: two
// scalar conversions shifted and or-ed together cost four instructions a pair.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  const f16x2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t u16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)u16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // round to nearest even
}

// Load one element of a tensor of runtime dtype as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case SIPA_F32: return ((const float*)p)[i];
    case SIPA_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    case SIPA_F16: return f16_bits_to_f32(((const uint16_t*)p)[i]);
    default: return (float)((const int8_t*)p)[i];
  }
}

__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dtype, float f) {
  switch (dtype) {
    case SIPA_F32: ((float*)p)[i] = f; break;
    case SIPA_BF16: ((uint16_t*)p)[i] = f32_to_bf16_bits(f); break;
    default: ((uint16_t*)p)[i] = f32_to_f16_bits(f); break;
  }
}

// ---- decode kernel arguments ---------------------------------------------------------------------------------

struct DecodeArgs {
  const void* q;
  int64_t q_ss, q_sh;
  const void* k;
  const void* v;
  int64_t kv_sh, kv_sn;
  const int32_t* bt;
  int64_t bt_ss;
  const int32_t* ctx;
  void* out;
  int64_t o_ss, o_sh;
  const void* ks;
  int64_t ks_sh, ks_sn;
  const void* vs;
  int64_t vs_sh, vs_sn;
  const void* stage;
  int64_t st_sh, st_sn, st_sb;
  const int32_t* tail;
  const int32_t* items;  // work list (8 int32 per workgroup), or NULL for the (sequence, KV head, split) grid
  float* part;        // [S, Hq, splits, D] unnormalised split outputs
  float* pm;          // [S, Hq, splits] split running max (log2 domain)
  float* pl;          // [S, Hq, splits] split softmax denominators
  int32_t* counters;  // [S, Hkv] splits finished, for the last-arriving merge
  int32_t S, Hq, Hkv, G, B, splits, chunk;
  int32_t chunk_old, n_old;  // the first n_old splits hold chunk_old tokens each, the rest chunk (n_old 0: uniform)
  int32_t max_ctx;    // every block-table row covers ceil(max_ctx / B) blocks; context lengths are clamped to it
  int32_t nb;         // blocks in the pool: block ids are clamped to [0, nb)
  int32_t bt_w;       // entries per block-table row (>= ceil(max_ctx / B)): table columns are clamped below it
  int32_t n_stage;    // staging slots (INT8 per-channel K): tail slots are clamped below it
  int32_t ks_f32, vs_f32;
  int32_t fused;      // 1: the last split workgroup of a (sequence, KV head) merges the splits
  float scale_log2;   // softmax scale * log2(e): scores are kept in the exp2 domain
};

// ---- host-side error reporting ---------------------------------------------------------------------------------

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

}  // namespace sipa

#define SIPA_CHECK(cond, code, ...)                       \
  do {                                                    \
    if (!(cond)) return ::sipa::fail((code), __VA_ARGS__); \
  } while (0)
