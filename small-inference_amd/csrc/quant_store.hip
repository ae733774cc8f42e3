// Fused INT8 quantize-and-store and plain scatter-store of new K/V tokens into the paged pool (gfx950).
//
// Quantizer (reference engine/quant.py:19-31, fused in engine/triton_quant.py:24-58), bit-exact:
//   s = fp16(absmax / 127)                 fp32 IEEE division, then round-to-nearest-even to fp16
//   q = s > 0 ? clamp(rint(x / float(s)), -127, 127) : 0      IEEE division, round-half-even
// hipcc lowers fp32 '/' to the correctly rounded v_div_scale / v_div_fmas / v_div_fixup sequence and rintf to
// v_rndne_f32; (_Float16) conversion rounds to nearest even. Nothing in this file is compiled with fast-math.
//
// Per-token (grid over (token, head) vectors): 16 lanes per vector, D/16 contiguous channels per lane, the absmax
// reduced with xor-shuffles inside the 16-lane group. Per-channel blocks (grid over (block, head) tiles): one
// lane per channel walks the block's B tokens, so every load instruction reads a contiguous row.
#include <algorithm>
#include <cmath>

#include "sipa_common.h"

namespace sipa {

constexpr float kQMax = 127.f;

__device__ __forceinline__ int8_t quantize_code(float x, float s32) {
  float q = (s32 > 0.f) ? rintf(x / s32) : 0.f;
  q = fminf(fmaxf(q, -kQMax), kQMax);
  return (int8_t)(int)q;
}

__device__ __forceinline__ float round_to_bf16(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

struct QTokArgs {
  const void* x;
  int64_t x_st, x_sh;
  const int64_t* blocks;
  const int64_t* offsets;
  int8_t* q;
  int64_t q_sh, q_sn;
  uint16_t* s;
  int64_t s_sh, s_sn;
  int32_t T, H, D, B, x_dtype;
  // a second pair (grid row blockIdx.y == 1) at the same slots, pools with the first pair's strides
  const void* x2;
  int64_t x2_st, x2_sh;
  int8_t* q2;
  uint16_t* s2;
};

template <int EPL>  // channels per lane: D / 16
__global__ void __launch_bounds__(256) quantize_tokens_kernel(const QTokArgs a) {
  const int vec = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (vec >= a.T * a.H) return;  // whole 16-lane groups leave together; shuffles stay inside a group
  const int t = vec / a.H, h = vec % a.H;
  const bool second = blockIdx.y != 0;
  const void* xs = second ? a.x2 : a.x;
  const int64_t xi = (int64_t)t * (second ? a.x2_st : a.x_st) + (int64_t)h * (second ? a.x2_sh : a.x_sh) + sub * EPL;
  float x[EPL];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    x[i] = load_as_f32(xs, xi + i, a.x_dtype);
    amax = fmaxf(amax, fabsf(x[i]));
  }
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const _Float16 sh = (_Float16)(amax / kQMax);
  const float s32 = (float)sh;
  const int64_t blk = a.blocks[t], off = a.offsets[t];
  int8_t* qrow = (second ? a.q2 : a.q) + (int64_t)h * a.q_sh + blk * a.q_sn + off * a.D + sub * EPL;
#pragma unroll
  for (int i = 0; i < EPL; ++i) qrow[i] = quantize_code(x[i], s32);
  if (sub == 0) (second ? a.s2 : a.s)[(int64_t)h * a.s_sh + blk * a.s_sn + off] = __builtin_bit_cast(uint16_t, sh);
}

struct QBlkArgs {
  const void* src;  // pool source [H, n_src, B, D] or rows source x [T, H, D]
  int64_t src_sh, src_sn, src_sb;
  const int64_t* src_idx;  // pool source: src[i]; rows source: rows[i * B + b]
  const int64_t* dst;
  int8_t* q;
  int64_t q_sh, q_sn;
  uint16_t* s;
  int64_t s_sh, s_sn;
  int32_t n, H, B, D, src_dtype, rows_mode;
};

__global__ void __launch_bounds__(256) quantize_blocks_kernel(const QBlkArgs a) {
  const int per_wg = 256 / a.D;  // (block, head) tiles per workgroup
  const int tile = blockIdx.x * per_wg + threadIdx.x / a.D;
  const int d = threadIdx.x % a.D;
  if (threadIdx.x >= per_wg * a.D || tile >= a.n * a.H) return;
  const int i = tile / a.H, h = tile % a.H;
  auto value = [&](int b) {
    int64_t idx;
    if (a.rows_mode)
      idx = a.src_idx[(int64_t)i * a.B + b] * a.src_sn + (int64_t)h * a.src_sh + d;
    else
      idx = (int64_t)h * a.src_sh + a.src_idx[i] * a.src_sn + (int64_t)b * a.src_sb + d;
    const float v = load_as_f32(a.src, idx, a.src_dtype);
    return a.rows_mode ? round_to_bf16(v) : v;  // the reference's cache quantizes the bf16-rounded K
  };
  const int64_t blk = a.dst[i];
  int8_t* qb = a.q + (int64_t)h * a.q_sh + blk * a.q_sn + d;
  float amax = 0.f;
  if (a.B == 16) {  // the paged block size: all 16 loads in flight at once, values kept in registers
    float v[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) v[b] = value(b);
#pragma unroll
    for (int b = 0; b < 16; ++b) amax = fmaxf(amax, fabsf(v[b]));
    const _Float16 sh = (_Float16)(amax / kQMax);
    const float s32 = (float)sh;
#pragma unroll
    for (int b = 0; b < 16; ++b) qb[(int64_t)b * a.D] = quantize_code(v[b], s32);
    a.s[(int64_t)h * a.s_sh + blk * a.s_sn + d] = __builtin_bit_cast(uint16_t, sh);
    return;
  }
  for (int b = 0; b < a.B; ++b) amax = fmaxf(amax, fabsf(value(b)));
  const _Float16 sh = (_Float16)(amax / kQMax);
  const float s32 = (float)sh;
  for (int b = 0; b < a.B; ++b) qb[(int64_t)b * a.D] = quantize_code(value(b), s32);  // second pass hits cache
  a.s[(int64_t)h * a.s_sh + blk * a.s_sn + d] = __builtin_bit_cast(uint16_t, sh);
}

struct StoreArgs {
  const void* x;
  const void* x2;
  int64_t x_st, x_sh;
  int64_t x2_st, x2_sh;
  const int64_t* rows;
  const int64_t* blocks;
  const int64_t* offsets;
  void* pool;
  void* pool2;
  int64_t p_sh, p_sn, p_sb;
  int32_t n, H, D, x_dtype, p_dtype;
};

__global__ void __launch_bounds__(256) store_tokens_kernel(const StoreArgs a) {
  const int64_t total = (int64_t)a.n * a.H * a.D;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int d = (int)(e % a.D);
    const int h = (int)((e / a.D) % a.H);
    const int i = (int)(e / ((int64_t)a.D * a.H));
    const int64_t row = a.rows ? a.rows[i] : i;
    const int64_t xi = row * a.x_st + (int64_t)h * a.x_sh + d;
    const int64_t pi = (int64_t)h * a.p_sh + a.blocks[i] * a.p_sn + a.offsets[i] * a.p_sb + d;
    store_from_f32(a.pool, pi, a.p_dtype, load_as_f32(a.x, xi, a.x_dtype));
    if (a.x2)
      store_from_f32(a.pool2, pi, a.p_dtype, load_as_f32(a.x2, row * a.x2_st + (int64_t)h * a.x2_sh + d, a.x_dtype));
  }
}

// Format B's writes of a decode step in one launch (sipa_kchan_write_rows): workgroup t takes row t's token.
//   V: per-token quantization at (blocks[t], offsets[t]), one 16-lane group per head, as quantize_tokens_kernel.
//   K: the bf16 rounding of k[t] into its staging slot at offsets[t], as store_tokens_kernel; then, when the row
//   quantizes its slot (dst[t] >= 0, or offsets[t] == B - 1 without dst), the slot's B tokens per channel into
//   block dst[t] (or blocks[t]), as quantize_blocks_kernel: token offsets[t] from the value just rounded, the
//   others from the slot, so nothing this launch stores is read back through memory.
struct KchanArgs {
  const void* k;
  const void* v;
  int64_t k_st, k_sh, v_st, v_sh;
  const int64_t* blocks;
  const int64_t* offsets;
  const int64_t* slots;
  const int64_t* dst;  // NULL: the row's own block when its offset is B - 1
  int8_t* vq;
  uint16_t* vs;
  int8_t* kq;
  uint16_t* ks;
  uint16_t* stage;
  int64_t q_sh, q_sn, vs_sh, vs_sn, ks_sh, ks_sn, st_sh, st_sn, st_sb;
  int32_t T, H, D, B, x_dtype;
};

template <int EPL>  // V channels per lane: D / 16
__global__ void __launch_bounds__(256) kchan_write_rows_kernel(const KchanArgs a) {
  const int t = blockIdx.x;
  const int64_t blk = a.blocks[t], off = a.offsets[t], slot = a.slots[t];
  // V: heads grp, grp + 16, ... of the row, 16 lanes each (whole 16-lane groups run each iteration together)
  const int grp = threadIdx.x >> 4, sub = threadIdx.x & 15;
  for (int h = grp; h < a.H; h += 16) {
    const int64_t xi = (int64_t)t * a.v_st + (int64_t)h * a.v_sh + sub * EPL;
    float x[EPL];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      x[i] = load_as_f32(a.v, xi + i, a.x_dtype);
      amax = fmaxf(amax, fabsf(x[i]));
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const _Float16 sh = (_Float16)(amax / kQMax);
    const float s32 = (float)sh;
    int8_t* qrow = a.vq + (int64_t)h * a.q_sh + blk * a.q_sn + off * a.D + sub * EPL;
#pragma unroll
    for (int i = 0; i < EPL; ++i) qrow[i] = quantize_code(x[i], s32);
    if (sub == 0) a.vs[(int64_t)h * a.vs_sh + blk * a.vs_sn + off] = __builtin_bit_cast(uint16_t, sh);
  }
  // K: one thread per (head, channel)
  const int64_t qdst = a.dst ? a.dst[t] : (off == a.B - 1 ? blk : -1);
  for (int e = threadIdx.x; e < a.H * a.D; e += 256) {
    const int h = e / a.D, d = e % a.D;
    const uint16_t kb = f32_to_bf16_bits(load_as_f32(a.k, (int64_t)t * a.k_st + (int64_t)h * a.k_sh + d, a.x_dtype));
    uint16_t* srow = a.stage + (int64_t)h * a.st_sh + slot * a.st_sn + d;  // token b of the slot at srow[b st_sb]
    srow[off * a.st_sb] = kb;
    if (qdst < 0) continue;
    auto value = [&](int b) { return bf16_bits_to_f32(b == off ? kb : srow[(int64_t)b * a.st_sb]); };
    int8_t* qb = a.kq + (int64_t)h * a.q_sh + qdst * a.q_sn + d;
    float amax = 0.f;
    if (a.B == 16) {  // the paged block size: all loads in flight at once, values kept in registers
      float v[16];
#pragma unroll
      for (int b = 0; b < 16; ++b) v[b] = value(b);
#pragma unroll
      for (int b = 0; b < 16; ++b) amax = fmaxf(amax, fabsf(v[b]));
      const _Float16 sh = (_Float16)(amax / kQMax);
      const float s32 = (float)sh;
#pragma unroll
      for (int b = 0; b < 16; ++b) qb[(int64_t)b * a.D] = quantize_code(v[b], s32);
      a.ks[(int64_t)h * a.ks_sh + qdst * a.ks_sn + d] = __builtin_bit_cast(uint16_t, sh);
      continue;
    }
    for (int b = 0; b < a.B; ++b) amax = fmaxf(amax, fabsf(value(b)));
    const _Float16 sh = (_Float16)(amax / kQMax);
    const float s32 = (float)sh;
    for (int b = 0; b < a.B; ++b) qb[(int64_t)b * a.D] = quantize_code(value(b), s32);
    a.ks[(int64_t)h * a.ks_sh + qdst * a.ks_sn + d] = __builtin_bit_cast(uint16_t, sh);
  }
}

static bool float_dtype(int dt) { return dt == SIPA_F32 || dt == SIPA_BF16 || dt == SIPA_F16; }

static int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIPA_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return SIPA_OK;
}

}  // namespace sipa

using namespace sipa;

static int quantize_tokens(const QTokArgs& a, void* stream) {
  const int T = a.T, H = a.H, D = a.D;
  if (T == 0) return SIPA_OK;
  SIPA_CHECK(T > 0 && H > 0, SIPA_EINVAL, "T %d, H %d", T, H);
  SIPA_CHECK(D > 0 && D % 16 == 0 && D <= 256, SIPA_EUNSUPPORTED, "head_dim %d must be a multiple of 16 <= 256", D);
  SIPA_CHECK(a.B > 0, SIPA_EINVAL, "block_size %d", a.B);
  SIPA_CHECK(float_dtype(a.x_dtype), SIPA_EUNSUPPORTED, "x dtype %d", a.x_dtype);
  SIPA_CHECK(a.x && a.blocks && a.offsets && a.q && a.s, SIPA_EINVAL, "NULL pointer");
  SIPA_CHECK(!a.x2 || (a.q2 && a.s2), SIPA_EINVAL, "the second pair needs both pools");
  const dim3 grid((unsigned)(((int64_t)T * H + 15) / 16), a.x2 ? 2 : 1);
  hipStream_t st = (hipStream_t)stream;
  switch (D / 16) {
    case 1: hipLaunchKernelGGL(quantize_tokens_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(quantize_tokens_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(quantize_tokens_kernel<4>, grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL(quantize_tokens_kernel<8>, grid, dim3(256), 0, st, a); break;
    case 16: hipLaunchKernelGGL(quantize_tokens_kernel<16>, grid, dim3(256), 0, st, a); break;
    default: return fail(SIPA_EUNSUPPORTED, "head_dim %d not in {16,32,64,128,256}", D);
  }
  return check_launch("quantize_store_tokens");
}

extern "C" int32_t sipa_quantize_store_tokens(const void* x, int32_t x_dtype, int64_t x_stride_t, int64_t x_stride_h,
                                              int32_t T, int32_t H, int32_t D, const int64_t* blocks,
                                              const int64_t* offsets, int8_t* q_pool, int64_t q_stride_h,
                                              int64_t q_stride_n, int32_t B, void* s_pool, int64_t s_stride_h,
                                              int64_t s_stride_n, void* stream) {
  QTokArgs a{x, x_stride_t, x_stride_h, blocks, offsets, q_pool, q_stride_h, q_stride_n,
             (uint16_t*)s_pool, s_stride_h, s_stride_n, T, H, D, B, x_dtype, nullptr, 0, 0, nullptr, nullptr};
  return quantize_tokens(a, stream);
}

extern "C" int32_t sipa_quantize_store_tokens_kv(const void* x, const void* x2, int32_t x_dtype, int64_t x_stride_t,
                                                 int64_t x_stride_h, int64_t x2_stride_t, int64_t x2_stride_h,
                                                 int32_t T, int32_t H, int32_t D, const int64_t* blocks,
                                                 const int64_t* offsets, int8_t* q_pool, int8_t* q_pool2,
                                                 int64_t q_stride_h, int64_t q_stride_n, int32_t B, void* s_pool,
                                                 void* s_pool2, int64_t s_stride_h, int64_t s_stride_n,
                                                 void* stream) {
  SIPA_CHECK(x2 != nullptr, SIPA_EINVAL, "NULL pointer");
  QTokArgs a{x, x_stride_t, x_stride_h, blocks, offsets, q_pool, q_stride_h, q_stride_n,
             (uint16_t*)s_pool, s_stride_h, s_stride_n, T, H, D, B, x_dtype,
             x2, x2_stride_t, x2_stride_h, q_pool2, (uint16_t*)s_pool2};
  return quantize_tokens(a, stream);
}

static int launch_blocks(const QBlkArgs& a, void* stream) {
  const int per_wg = 256 / a.D;
  const dim3 grid((unsigned)(((int64_t)a.n * a.H + per_wg - 1) / per_wg));
  hipLaunchKernelGGL(quantize_blocks_kernel, grid, dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("quantize_store_blocks");
}

extern "C" int32_t sipa_quantize_store_blocks(const void* src_pool, int32_t src_dtype, int64_t src_stride_h,
                                              int64_t src_stride_n, int64_t src_stride_b, const int64_t* src,
                                              const int64_t* dst, int32_t n, int32_t H, int32_t B, int32_t D,
                                              int8_t* q_pool, int64_t q_stride_h, int64_t q_stride_n, void* s_pool,
                                              int64_t s_stride_h, int64_t s_stride_n, void* stream) {
  if (n == 0) return SIPA_OK;
  SIPA_CHECK(n > 0 && H > 0, SIPA_EINVAL, "n %d, H %d", n, H);
  SIPA_CHECK(D > 0 && D <= 256 && 256 % D == 0, SIPA_EUNSUPPORTED, "head_dim %d must divide 256", D);
  SIPA_CHECK(B > 0 && B <= 64, SIPA_EUNSUPPORTED, "block_size %d must be in [1, 64]", B);
  SIPA_CHECK(float_dtype(src_dtype), SIPA_EUNSUPPORTED, "source dtype %d", src_dtype);
  SIPA_CHECK(src_pool && src && dst && q_pool && s_pool, SIPA_EINVAL, "NULL pointer");
  QBlkArgs a{src_pool, src_stride_h, src_stride_n, src_stride_b, src, dst, q_pool, q_stride_h, q_stride_n,
             (uint16_t*)s_pool, s_stride_h, s_stride_n, n, H, B, D, src_dtype, 0};
  return launch_blocks(a, stream);
}

extern "C" int32_t sipa_quantize_store_block_rows(const void* x, int32_t x_dtype, int64_t x_stride_t,
                                                  int64_t x_stride_h, const int64_t* rows, const int64_t* dst,
                                                  int32_t n, int32_t H, int32_t B, int32_t D, int8_t* q_pool,
                                                  int64_t q_stride_h, int64_t q_stride_n, void* s_pool,
                                                  int64_t s_stride_h, int64_t s_stride_n, void* stream) {
  if (n == 0) return SIPA_OK;
  SIPA_CHECK(n > 0 && H > 0, SIPA_EINVAL, "n %d, H %d", n, H);
  SIPA_CHECK(D > 0 && D <= 256 && 256 % D == 0, SIPA_EUNSUPPORTED, "head_dim %d must divide 256", D);
  SIPA_CHECK(B > 0 && B <= 64, SIPA_EUNSUPPORTED, "block_size %d must be in [1, 64]", B);
  SIPA_CHECK(float_dtype(x_dtype), SIPA_EUNSUPPORTED, "x dtype %d", x_dtype);
  SIPA_CHECK(x && rows && dst && q_pool && s_pool, SIPA_EINVAL, "NULL pointer");
  QBlkArgs a{x, x_stride_h, x_stride_t, 0, rows, dst, q_pool, q_stride_h, q_stride_n,
             (uint16_t*)s_pool, s_stride_h, s_stride_n, n, H, B, D, x_dtype, 1};
  return launch_blocks(a, stream);
}

extern "C" int32_t sipa_store_tokens(const void* x, const void* x2, int32_t x_dtype, int64_t x_stride_t,
                                     int64_t x_stride_h, int64_t x2_stride_t, int64_t x2_stride_h,
                                     const int64_t* rows, int32_t n, int32_t H, int32_t D,
                                     const int64_t* blocks, const int64_t* offsets, void* pool, void* pool2,
                                     int32_t pool_dtype, int64_t p_stride_h, int64_t p_stride_n, int64_t p_stride_b,
                                     void* stream) {
  if (n == 0) return SIPA_OK;
  SIPA_CHECK(n > 0 && H > 0 && D > 0, SIPA_EINVAL, "n %d, H %d, D %d", n, H, D);
  SIPA_CHECK(float_dtype(x_dtype) && float_dtype(pool_dtype), SIPA_EUNSUPPORTED, "dtypes %d -> %d", x_dtype,
             pool_dtype);
  SIPA_CHECK(x && blocks && offsets && pool, SIPA_EINVAL, "NULL pointer");
  SIPA_CHECK((x2 == nullptr) == (pool2 == nullptr), SIPA_EINVAL, "x2 and pool2 go together");
  StoreArgs a{x, x2, x_stride_t, x_stride_h, x2_stride_t, x2_stride_h, rows, blocks, offsets, pool, pool2,
              p_stride_h, p_stride_n, p_stride_b, n, H, D, x_dtype, pool_dtype};
  const int64_t total = (int64_t)n * H * D;
  const unsigned wgs = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(store_tokens_kernel, dim3(wgs), dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("store_tokens");
}

extern "C" int32_t sipa_kchan_write_rows(const sipa_kchan_write_params* p, void* stream) {
  SIPA_CHECK(p != nullptr, SIPA_EINVAL, "NULL parameter block");
  if (p->T == 0) return SIPA_OK;
  SIPA_CHECK(p->T > 0 && p->H > 0, SIPA_EINVAL, "T %d, H %d", p->T, p->H);
  SIPA_CHECK(p->D > 0 && p->D % 16 == 0 && p->D <= 256, SIPA_EUNSUPPORTED, "head_dim %d must be a multiple of 16 <= 256",
             p->D);
  SIPA_CHECK(p->B > 0 && p->B <= 64, SIPA_EUNSUPPORTED, "block_size %d must be in [1, 64]", p->B);
  SIPA_CHECK(float_dtype(p->x_dtype), SIPA_EUNSUPPORTED, "k/v dtype %d", p->x_dtype);
  SIPA_CHECK(p->k && p->v && p->blocks && p->offsets && p->stage_slots && p->v_pool && p->v_scale && p->k_pool &&
                 p->k_scale && p->stage,
             SIPA_EINVAL, "NULL pointer");
  KchanArgs a{p->k, p->v, p->k_stride_t, p->k_stride_h, p->v_stride_t, p->v_stride_h, p->blocks, p->offsets,
              p->stage_slots, p->quant_dst, p->v_pool, (uint16_t*)p->v_scale, p->k_pool, (uint16_t*)p->k_scale,
              (uint16_t*)p->stage, p->q_stride_h, p->q_stride_n, p->vs_stride_h, p->vs_stride_n, p->ks_stride_h,
              p->ks_stride_n, p->st_stride_h, p->st_stride_n, p->st_stride_b, p->T, p->H, p->D, p->B, p->x_dtype};
  const dim3 grid((unsigned)p->T);
  hipStream_t st = (hipStream_t)stream;
  switch (p->D / 16) {
    case 1: hipLaunchKernelGGL(kchan_write_rows_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(kchan_write_rows_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(kchan_write_rows_kernel<4>, grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL(kchan_write_rows_kernel<8>, grid, dim3(256), 0, st, a); break;
    case 16: hipLaunchKernelGGL(kchan_write_rows_kernel<16>, grid, dim3(256), 0, st, a); break;
    default: return fail(SIPA_EUNSUPPORTED, "head_dim %d not in {16,32,64,128,256}", p->D);
  }
  return check_launch("kchan_write_rows");
}
