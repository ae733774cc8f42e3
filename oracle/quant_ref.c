/*
 * oracle/quant_ref.c -- TEST INFRASTRUCTURE ONLY. A CPU restatement, in plain C, of the reference's symmetric
 * absmax INT8 quantizer with fp16 scales. Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline may
 * load it, and only as the checker; the product never calls it.
 *
 * Follows reference engine/quant.py:19-31 (QMAX, _scale, _quantize), which engine/triton_quant.py:32-35,53-56
 * reproduces on the GPU:
 *   scale = fp16(absmax / 127)       absmax in fp32, IEEE binary32 division, round-to-nearest-even to binary16
 *   code  = scale > 0 ? clamp(round_half_even(x / float(scale)), -127, 127) : 0     IEEE binary32 division
 *
 * Built with gcc -O2 and no fast-math (x86-64 SSE arithmetic is IEEE binary32 with FLT_EVAL_METHOD 0; rintf in
 * the default rounding mode rounds half to even). The binary16 conversion is written out below because gcc 11
 * has no _Float16 on x86-64.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint32_t bits_of(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

static float float_of(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* binary32 -> binary16, round to nearest, ties to even; overflow to inf; NaN stays NaN. */
uint16_t oracle_f32_to_f16(float f) {
  const uint32_t x = bits_of(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);   /* NaN */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* >= 65520 (and inf) round to inf */
  if (ax < 0x38800000u) {
    /* below 2^-14: a multiple of the subnormal unit 2^-24. Scaling by 2^24 is exact; rintf rounds half to even;
       a result of 1024 is the smallest normal, whose bit pattern 0x0400 is the same integer. */
    return (uint16_t)(sign | (uint16_t)rintf(float_of(ax) * 16777216.0f));
  }
  const uint32_t mant = ax & 0x7fffffu;
  const uint32_t exp16 = (ax >> 23) - 127u + 15u;
  uint32_t h = (exp16 << 10) | (mant >> 13);
  const uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u; /* a carry into the exponent is still correct */
  return (uint16_t)(sign | h);
}

/* binary16 -> binary32 (exact). */
float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
    return float_of(bits_of(v) | sign);
  }
  if (e == 31) return float_of(sign | 0x7f800000u | (m << 13));
  return float_of(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

/*
 * Quantize n_groups groups of group_len values. Element i of group g is x[g * group_stride + i * elem_stride];
 * its code goes to the same index of q and the group's fp16 scale bits to scales[g]. Per token: groups are the
 * D channels of a (token, head); per channel: groups are one channel's B tokens of a block.
 */
void oracle_quantize_groups(const float* x, int64_t n_groups, int64_t group_len, int64_t group_stride,
                            int64_t elem_stride, int8_t* q, uint16_t* scales) {
  for (int64_t g = 0; g < n_groups; ++g) {
    const float* xg = x + g * group_stride;
    float absmax = 0.0f;
    for (int64_t i = 0; i < group_len; ++i) {
      const float a = fabsf(xg[i * elem_stride]);
      if (a > absmax) absmax = a;
    }
    const uint16_t s16 = oracle_f32_to_f16(absmax / 127.0f);
    const float s = oracle_f16_to_f32(s16);
    scales[g] = s16;
    for (int64_t i = 0; i < group_len; ++i) {
      float c = 0.0f;
      if (s > 0.0f) {
        c = rintf(xg[i * elem_stride] / s);
        if (c > 127.0f) c = 127.0f;
        if (c < -127.0f) c = -127.0f;
      }
      q[g * group_stride + i * elem_stride] = (int8_t)c;
    }
  }
}
