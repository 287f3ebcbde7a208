/*
 * kq_oracle.c -- CPU restatement of Kshipra's weight-only quantized linear
 * path (engine/quantization.py), in plain C with IEEE-754 binary32 arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it and never
 * falls back to it.
 *
 * Every function cites the reference lines it restates.  The arithmetic is a
 * closed form (true division, round-half-to-even, fp32 -> fp16 round-to-
 * nearest-even with subnormals), so the outputs are bit-determined.
 * Build: gcc -O2 -std=c11 -fno-fast-math -ffp-contract=off -fPIC -shared
 * (x86-64 SSE2: FLT_EVAL_METHOD == 0, so float ops round to binary32).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(FLT_EVAL_METHOD) && FLT_EVAL_METHOD != 0
#error "binary32 expressions must be evaluated in binary32"
#endif

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary32 -> binary16, round to nearest, ties to even, with subnormals,
 * overflow to infinity and NaN kept quiet.  This is the conversion torch's
 * Tensor.to(torch.float16) performs (engine/quantization.py:208, :295). */
uint16_t kqo_f32_to_f16(float f) {
  uint32_t x = f32_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);           /* NaN */
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* >= 65520 -> inf */
  uint32_t e = ax >> 23;                                              /* biased fp32 exponent */
  uint32_t m = (ax & 0x7FFFFFu);
  if (e >= 113u) {                                                    /* |f| >= 2^-14: normal fp16 */
    uint32_t h = ((e - 112u) << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;           /* carry may bump exponent */
    return (uint16_t)(sign | h);
  }
  if (e == 0u) return (uint16_t)sign;                                 /* fp32 subnormal -> +-0 */
  /* fp16 subnormal: value / 2^-24 = (m | 2^23) * 2^(e - 126), e <= 112 */
  uint32_t mant = m | 0x800000u;
  uint32_t shift = 126u - e;                                          /* >= 14 */
  if (shift > 24u) return (uint16_t)sign;                             /* < 2^-25: rounds to 0 */
  uint32_t h = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

/* binary16 -> binary32 (exact). */
float kqo_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t m = (uint32_t)h & 0x3FFu;
  if (e == 0x1Fu) return bits_f32(sign | 0x7F800000u | (m << 13));
  if (e == 0u) {
    if (m == 0u) return bits_f32(sign);
    float v = (float)m * 5.9604644775390625e-08f;                     /* m * 2^-24, exact */
    return (sign ? -v : v);
  }
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* torch.round(t).clamp(lo, hi).to(torch.int8): rint is half-to-even; NaN
 * survives clamp and the NaN -> int8 cast yields 0 (torch CPU behaviour);
 * +-inf clamps to the range ends. */
static int8_t round_clamp(float t, float lo, float hi) {
  if (isnan(t)) return 0;
  float r = rintf(t);
  if (r < lo) r = lo;
  if (r > hi) r = hi;
  return (int8_t)r;
}

/* engine/quantization.py:196-223  quantize_int8_per_channel (after the
 * _validate_weight checks at :180-188, which the caller performs). */
void kqo_quantize_int8(const float* w, int64_t n, int64_t k, int64_t ldw,
                       int8_t* q, uint16_t* s) {
  for (int64_t r = 0; r < n; r++) {
    const float* row = w + r * ldw;
    float m = 0.0f;                                                   /* :206 abs().amax(dim=1) */
    for (int64_t c = 0; c < k; c++) { float a = fabsf(row[c]); if (a > m) m = a; }
    float s32 = m / 127.0f;                                           /* :207 true division */
    if (s32 < 1e-8f) s32 = 1e-8f;                                     /* :207 clamp_min(1e-8) */
    uint16_t h = kqo_f32_to_f16(s32);                                 /* :208 */
    s[r] = h;
    float sq = kqo_f16_to_f32(h);                                     /* :215 */
    for (int64_t c = 0; c < k; c++)                                   /* :216-217 */
      q[r * k + c] = round_clamp(row[c] / sq, -127.0f, 127.0f);
  }
}

/* engine/quantization.py:226-230  _dequantize_int8_per_channel (exact). */
void kqo_dequantize_int8(const int8_t* q, const uint16_t* s, int64_t n, int64_t k, float* out) {
  for (int64_t r = 0; r < n; r++) {
    float sc = kqo_f16_to_f32(s[r]);
    for (int64_t c = 0; c < k; c++) out[r * k + c] = (float)q[r * k + c] * sc;
  }
}

/* engine/quantization.py:238-318  quantize_int4_per_group.  group_size must
 * be positive and even (checked by the caller, :273-276).  Columns past k are
 * the zero padding of :283-290.  Packing :304-309: low nibble = even index. */
void kqo_quantize_int4(const float* w, int64_t n, int64_t k, int64_t ldw, int64_t g,
                       uint8_t* q, uint16_t* s) {
  int64_t ng = (k + g - 1) / g;
  int64_t kp = ng * g;
  for (int64_t r = 0; r < n; r++) {
    const float* row = w + r * ldw;
    for (int64_t gi = 0; gi < ng; gi++) {
      int64_t c0 = gi * g, c1 = c0 + g;
      float m = 0.0f;                                                 /* :293 (padding is 0) */
      for (int64_t c = c0; c < c1 && c < k; c++) { float a = fabsf(row[c]); if (a > m) m = a; }
      float s32 = m / 7.0f;                                           /* :294 */
      if (s32 < 1e-8f) s32 = 1e-8f;
      uint16_t h = kqo_f32_to_f16(s32);                               /* :295, :313 */
      s[r * ng + gi] = h;
      float sq = kqo_f16_to_f32(h);                                   /* :298 */
      for (int64_t c = c0; c < c1; c++) {
        float v = (c < k) ? row[c] : 0.0f;
        uint8_t u = (uint8_t)round_clamp(v / sq, -8.0f, 7.0f) & 0x0Fu;  /* :299-307 */
        uint8_t* byte = q + r * (kp / 2) + c / 2;
        if ((c & 1) == 0) *byte = u;                                  /* :309 low nibble */
        else *byte = (uint8_t)(*byte | (u << 4));                     /* :309 high nibble */
      }
    }
  }
}

/* engine/quantization.py:321-344  _dequantize_int4_per_group (exact), first
 * k of the kp padded columns. */
void kqo_dequantize_int4(const uint8_t* q, const uint16_t* s, int64_t n, int64_t k,
                         int64_t g, int64_t kp, float* out) {
  int64_t ng = kp / g;
  for (int64_t r = 0; r < n; r++) {
    for (int64_t c = 0; c < k; c++) {
      uint8_t b = q[r * (kp / 2) + c / 2];
      int u = (c & 1) ? ((b >> 4) & 0xF) : (b & 0xF);                 /* :328-333 */
      int v = (u >= 8) ? u - 16 : u;                                  /* :335 */
      out[r * k + c] = (float)v * kqo_f16_to_f32(s[r * ng + c / g]);  /* :337-343 */
    }
  }
}

/* Count of non-finite entries (engine/quantization.py:187). */
int64_t kqo_count_nonfinite(const float* w, int64_t n, int64_t k, int64_t ldw) {
  int64_t bad = 0;
  for (int64_t r = 0; r < n; r++)
    for (int64_t c = 0; c < k; c++) bad += !isfinite(w[r * ldw + c]);
  return bad;
}
