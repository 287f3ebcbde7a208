// Shared device/host helpers for the gfx950 quantized-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/kshipra_quant.h"

// ---------------------------------------------------------------------------
// Host-side status plumbing (defined in kq_capi.hip)
// ---------------------------------------------------------------------------
int kq_set_error(int status, const std::string& msg);
int kq_check_launch(const char* what);

#define KQ_REQUIRE(cond, msg)                                   \
  do {                                                          \
    if (!(cond)) return kq_set_error(KQ_ERR_ARG, (msg));        \
  } while (0)

static inline hipStream_t kq_stream(kq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------
// Vector types
// ---------------------------------------------------------------------------
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// fp32 -> fp16, round to nearest even, subnormals kept (v_cvt_f16_f32 under the
// default gfx950 mode: RNE, fp16 denormals enabled).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int DT>
__device__ __forceinline__ float load_f32(const void* p, int64_t i);
template <>
__device__ __forceinline__ float load_f32<KQ_F32>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <>
__device__ __forceinline__ float load_f32<KQ_F16>(const void* p, int64_t i) {
  return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <>
__device__ __forceinline__ float load_f32<KQ_BF16>(const void* p, int64_t i) {
  return __builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(p)[i] << 16);
}

// torch.round(t).clamp(lo, hi).to(int8): rint is round-half-to-even; NaN
// passes clamp and casts to 0 (torch CPU); +-inf clamps to the range ends.
__device__ __forceinline__ int round_clamp(float t, float lo, float hi) {
  if (__builtin_isnan(t)) return 0;
  float r = __builtin_rintf(t);
  r = __builtin_fmaxf(r, lo);
  r = __builtin_fminf(r, hi);
  return (int)r;
}

// ---------------------------------------------------------------------------
// Wavefront reductions (64 lanes)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// DPP lane moves (gfx9 encodings of dpp_ctrl): quad permutations, the
// half-row / row mirrors and the row broadcasts of lane 15 / 31.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move(float v) {
  const int i = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(i, i, CTRL, ROW_MASK, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;          // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;   // lane i <- 7 - i within 8
constexpr int kDppMirror = 0x140;       // lane i <- 15 - i within 16
constexpr int kDppBcast15 = 0x142;      // row r <- lane 15 of row r - 1
constexpr int kDppBcast31 = 0x143;      // rows 2, 3 <- lane 31

// Maximum over aligned groups of g lanes (g = 4, 8, 16, 32 or 64), returned
// to every lane of the group.  Masked-off lanes keep their own value, which
// leaves the maximum unchanged.
__device__ __forceinline__ float group_max(float v, int g) {
  v = __builtin_fmaxf(v, dpp_move<kDppXor1>(v));
  v = __builtin_fmaxf(v, dpp_move<kDppXor2>(v));
  if (g > 4) v = __builtin_fmaxf(v, dpp_move<kDppHalfMirror>(v));
  if (g > 8) v = __builtin_fmaxf(v, dpp_move<kDppMirror>(v));
  if (g > 16) v = __builtin_fmaxf(v, __shfl_xor(v, 16, 64));
  if (g > 32) v = __builtin_fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// Maximum over the whole wave as a wave-uniform value: reduce within rows of
// 16, then carry row maxima upward with the row broadcasts; lane 63 ends with
// the total.
__device__ __forceinline__ float wave_max_uniform(float v) {
  v = __builtin_fmaxf(v, dpp_move<kDppXor1>(v));
  v = __builtin_fmaxf(v, dpp_move<kDppXor2>(v));
  v = __builtin_fmaxf(v, dpp_move<kDppHalfMirror>(v));
  v = __builtin_fmaxf(v, dpp_move<kDppMirror>(v));
  v = __builtin_fmaxf(v, dpp_move<kDppBcast15, 0xa>(v));
  v = __builtin_fmaxf(v, dpp_move<kDppBcast31, 0xc>(v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------------------
// Packed-weight -> fp16 MFMA operand conversions (exact)
//
// INT4: one 32-bit word holds 8 two's-complement nibbles, nibble p = bits
// [4p, 4p+4) = column 8i+p of the 16-byte chunk's word i.  XOR 0x8 turns each
// nibble into u = q + 8 in [0, 15]; OR-ing it under the fp16 exponent of 1024
// gives 1024 + u (bits 0-3) or 1024 + 16u (bits 4-7), exact; one packed fp16
// add / fma removes the bias.  Output halves, in order:
//   [q0, q4, q1, q5, q2, q6, q3, q7]  (slot s <-> nibble kPermInt4[s])
// ---------------------------------------------------------------------------
// The three constants a VOP3 instruction cannot take beside its one scalar
// operand (the nibble masks and -72): a loop can hold them in VGPRs
// (int4_consts_pinned) instead of rebuilding them for every word.
struct Int4Consts {
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, b1 = 0xD480D480u;   // b1: (-72, -72) in fp16
};
__device__ __forceinline__ Int4Consts int4_consts_pinned() {
  Int4Consts k;
  __asm__ volatile("" : "+v"(k.mlo), "+v"(k.mhi), "+v"(k.b1));
  return k;
}

__device__ __forceinline__ half8_t int4x8_to_half8(uint32_t w, const Int4Consts& k = Int4Consts{}) {
  // ((w ^ 0x88888888) & M) | 0x6400_6400 == (w & M) ^ (0x6400_6400 | (0x88888888 & M))
  const uint32_t w8 = w >> 8;
  const half2_t t0 = __builtin_bit_cast(half2_t, (w & k.mlo) ^ 0x64086408u);
  const half2_t t1 = __builtin_bit_cast(half2_t, (w & k.mhi) ^ 0x64806480u);
  const half2_t t2 = __builtin_bit_cast(half2_t, (w8 & k.mlo) ^ 0x64086408u);
  const half2_t t3 = __builtin_bit_cast(half2_t, (w8 & k.mhi) ^ 0x64806480u);
  const half2_t b0 = {(_Float16)1032.0f, (_Float16)1032.0f};
  const half2_t m1 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2_t b1 = __builtin_bit_cast(half2_t, k.b1);
  const half2_t r0 = t0 - b0;
  const half2_t r1 = t1 * m1 + b1;
  const half2_t r2 = t2 - b0;
  const half2_t r3 = t3 * m1 + b1;
  half8_t o;
  o[0] = r0[0]; o[1] = r0[1]; o[2] = r1[0]; o[3] = r1[1];
  o[4] = r2[0]; o[5] = r2[1]; o[6] = r3[0]; o[7] = r3[1];
  return o;
}

// INT8: two words = 8 two's-complement bytes b0..b7.  XOR 0x80 gives
// u = q + 128 in [0, 255]; v_perm places u under the fp16 exponent of 1024
// (0x64), giving 1024 + u exactly; a packed fp16 add of -1152 yields q.
// Output halves: [q0, q2, q1, q3, q4, q6, q5, q7] (slot s <-> byte kPermInt8[s]).
__device__ __forceinline__ half8_t int8x8_to_half8(uint32_t w0, uint32_t w1) {
  const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
  const uint32_t k64 = 0x64646464u;
  const half2_t t0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(k64, x0, 0x04020400u));
  const half2_t t1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(k64, x0, 0x04030401u));
  const half2_t t2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(k64, x1, 0x04020400u));
  const half2_t t3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(k64, x1, 0x04030401u));
  const half2_t b = {(_Float16)1152.0f, (_Float16)1152.0f};
  const half2_t r0 = t0 - b, r1 = t1 - b, r2 = t2 - b, r3 = t3 - b;
  half8_t o;
  o[0] = r0[0]; o[1] = r0[1]; o[2] = r1[0]; o[3] = r1[1];
  o[4] = r2[0]; o[5] = r2[1]; o[6] = r3[0]; o[7] = r3[1];
  return o;
}

// Slot -> column offset within the 8 columns an operand slot group covers.
__host__ __device__ constexpr int perm_int4(int s) { return (s & 1) ? 4 + (s >> 1) : (s >> 1); }
__host__ __device__ constexpr int perm_int8(int s) {
  return (s & 4) | (((s & 1) << 1) | ((s & 2) >> 1));
}

// ---------------------------------------------------------------------------
// MFMA operand geometry (v_mfma_f32_16x16x32_f16, wave64)
//
// One MFMA "k-step" T contracts 32 columns.  Lane l = 16*qd + c supplies
// A row c and B column c at k-slots 8*qd .. 8*qd+7.  The 32 columns of
// k-step T, lane quad qd, slot s are:
//   INT4 (group g = T/4, i = T%4):  128g + 32qd + 8i + perm_int4(s)
//   INT8 (window w = T/2, j = T%2):  64w + 16qd + 8j + perm_int8(s)
// so a lane's 16-byte weight load (INT4: one quarter of a 128-column group;
// INT8: one quarter of a 64-column window) feeds 4 (INT4) or 2 (INT8)
// consecutive k-steps.  The activation operand uses the same map; it is
// staged as fp16 hi/lo pairs of the power-of-two scaled activation
// (x 2^e = hi + lo, hi = fp16(x 2^e), lo = fp16(x 2^e - hi); see below).
// ---------------------------------------------------------------------------
template <int BITS>
__host__ __device__ constexpr int64_t kstep_col0(int64_t T, int qd) {
  return BITS == 4 ? 128 * (T >> 2) + 32 * qd + 8 * (T & 3)
                   : 64 * (T >> 1) + 16 * qd + 8 * (T & 1);
}
template <int BITS>
__host__ __device__ constexpr int kstep_perm(int s) {
  return BITS == 4 ? perm_int4(s) : perm_int8(s);
}

__device__ __forceinline__ floatx4 mfma16x16x32(half8_t a, half8_t b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Range-safe activation split.
//
// fp16 covers 2^-24 .. 65504; fp32 activations span 2^-149 .. 2^128.  A row
// of x (or the K-slice of a row that one accumulation chain covers) is
// therefore scaled by an exact power of two 2^e, chosen from its largest
// magnitude so that max |x| * 2^e lies in [2^14, 2^15), before it is split
// into hi = fp16(x 2^e) and lo = fp16(x 2^e - hi).  The products of exact
// fp16 weights with hi / lo are exact in the fp32 accumulators, and the sum
// is scaled back by 2^-e (exact unless the result itself leaves the fp32
// range).  The representation error of an element is at most 2^-22 |x| (hi
// keeps 11 bits, lo the next 11) plus 2^-25 in the scaled domain (lo's
// subnormal spacing), i.e. 2^-39 of the slice maximum: fp32-class for every
// finite x, whatever its magnitude.  (A staging path may scale by up to 12
// below the optimal exponent -- max |x| * 2^e in [2^2, 2^15) -- which moves
// that floor to 2^-27 of the maximum and leaves the 2^-22 |x| term.)
//
// Non-finite entries: the maximum is taken over |x| with NaN ignored and is
// clamped to FLT_MAX, so a row holding +-inf keeps its finite entries in
// range; +-inf itself becomes hi = +-inf, lo = 0 (products inf * q give
// +-inf, or NaN for q = 0, as the fp32 product does); NaN stays NaN.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float absmax8(const float (&v)[8], float m) {
#pragma unroll
  for (int s = 0; s < 8; s++) m = __builtin_fmaxf(m, __builtin_fabsf(v[s]));
  return m;
}

// Scale exponent of a row-slice whose largest magnitude is amax (>= 0):
// amax * 2^e in [2^14, 2^15); 0 for an all-zero (or all-NaN) slice.
__device__ __forceinline__ int act_exponent(float amax) {
  amax = __builtin_fminf(amax, 3.40282347e38f);
  return amax > 0.0f ? 15 - __builtin_amdgcn_frexp_expf(amax) : 0;
}

// Split 8 fp32 activations (already in slot order) scaled by 2^e into fp16
// hi/lo halves.  Per pair: hi = both halves rounded in one packed conversion;
// lo = fp16(fma(hi, -1, t)), the exact remainder rounded once, written into
// the low / high half by the mixed-precision fma (op_sel picks hi's half).
// guard: wave-uniform, true when some lane of the wave may split a +-inf
// entry (its running max |x| is inf).  Such an entry has hi = +-inf and
// lo = inf - inf = NaN; the guarded fix-up makes that lo 0.  (lo must be 0,
// not merely finite: a large finite lo-row sum scaled back by 2^-e could
// itself overflow and meet hi's inf with the opposite sign.)  A finite t has
// |t| < 2^15, so hi = +-inf marks exactly the infinite entries; NaN stays NaN.
__device__ __forceinline__ void split_hi_lo(const float (&v)[8], int e, half8_t& hi, half8_t& lo,
                                            bool guard) {
  u32x4 h4, l4;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const float t0 = __builtin_amdgcn_ldexpf(v[2 * p], e);
    const float t1 = __builtin_amdgcn_ldexpf(v[2 * p + 1], e);
    uint32_t h2, l2;
    __asm__("v_cvt_pk_f16_f32 %0, %2, %3\n\t"
            "v_fma_mixlo_f16 %1, %0, -1.0, %2 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mixhi_f16 %1, %0, -1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "=&v"(h2), "=&v"(l2)
            : "v"(t0), "v"(t1));
    h4[p] = h2;
    l4[p] = l2;
  }
  hi = __builtin_bit_cast(half8_t, h4);
  lo = __builtin_bit_cast(half8_t, l4);
  if (guard) {
#pragma unroll
    for (int s = 0; s < 8; s++)
      if (__builtin_isinf((float)hi[s])) lo[s] = (_Float16)0.0f;
  }
}

// Wave-uniform guard for split_hi_lo from each lane's running max |x| over
// the entries it converts.
__device__ __forceinline__ bool wave_has_inf(float lane_amax) {
  return __builtin_amdgcn_ballot_w64(lane_amax == __builtin_inff()) != 0;
}

// Undo the activation scale on an fp32 (partial) sum.
__device__ __forceinline__ float unscale(float v, int e) { return __builtin_amdgcn_ldexpf(v, -e); }
