// Quantize / pack / dequantize kernels (gfx950).
//
// Bit-exact restatements of Kshipra engine/quantization.py:
//   quantize_int8_per_channel   :196-223   -> q8_rows_kernel
//   quantize_int4_per_group     :238-318   -> q4_groups_kernel
//   _dequantize_int8_per_channel :226-230  -> dq8_kernel
//   _dequantize_int4_per_group  :321-344   -> dq4_kernel
//   _validate_weight isfinite   :187       -> finite_kernel
//
// These run once per weight at load time and are HBM-bound byte work: each
// weight is read twice (max pass, quantize pass; the second read of a row or
// group is an L2 hit) and written once as 1 byte or half a byte.
#include "kq_common.hpp"

namespace {

constexpr int kQ8Threads = 256;

// One workgroup per output row (grid-stride).  Pass 1: |w| max and the
// non-finite flag over the row.  Pass 2: q = rint(w / fp16(s)).
template <int DT>
__global__ __launch_bounds__(kQ8Threads) void q8_rows_kernel(const void* __restrict__ w, int64_t n,
                                                             int64_t k, int64_t ldw,
                                                             int8_t* __restrict__ q,
                                                             uint16_t* __restrict__ s,
                                                             int32_t* __restrict__ flag) {
  __shared__ float red_max[kQ8Threads / 64];
  __shared__ int red_bad[kQ8Threads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  for (int64_t r = blockIdx.x; r < n; r += gridDim.x) {
    const int64_t base = r * ldw;
    float m = 0.0f;
    int bad = 0;
    for (int64_t c = tid; c < k; c += kQ8Threads) {
      const float v = load_f32<DT>(w, base + c);
      bad |= !__builtin_isfinite(v);
      m = __builtin_fmaxf(m, __builtin_fabsf(v));
    }
    m = wave_max(m);
    bad = wave_or(bad);
    if (lane == 0) { red_max[wv] = m; red_bad[wv] = bad; }
    __syncthreads();
    m = red_max[0];
    bad = red_bad[0];
#pragma unroll
    for (int i = 1; i < kQ8Threads / 64; i++) { m = __builtin_fmaxf(m, red_max[i]); bad |= red_bad[i]; }
    __syncthreads();
    if (bad && tid == 0) flag[0] = 1;
    float s32 = m / 127.0f;                          // :207 true division
    s32 = s32 < 1e-8f ? 1e-8f : s32;                 // :207 clamp_min(1e-8)
    const uint16_t h = f32_to_f16_bits(s32);         // :208
    const float sq = f16_bits_to_f32(h);             // :215
    if (tid == 0) s[r] = h;
    for (int64_t c = tid; c < k; c += kQ8Threads) {  // :216-217
      const float v = load_f32<DT>(w, base + c);
      q[r * k + c] = (int8_t)round_clamp(v / sq, -127.0f, 127.0f);
    }
  }
}

// One wavefront per (row, group) unit (grid-stride).  Lane j owns column pairs
// (2j, 2j+1), (2j+128, 2j+129), ... of the group and writes their packed byte.
template <int DT>
__global__ __launch_bounds__(256) void q4_groups_kernel(const void* __restrict__ w, int64_t n,
                                                        int64_t k, int64_t ldw, int64_t g,
                                                        int64_t ng, uint8_t* __restrict__ q,
                                                        uint16_t* __restrict__ s,
                                                        int32_t* __restrict__ flag) {
  const int lane = threadIdx.x & 63;
  const int64_t units = n * ng;
  const int64_t wave0 = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * (blockDim.x >> 6);
  const int64_t row_bytes = ng * g / 2;
  for (int64_t u = wave0; u < units; u += wstride) {
    const int64_t r = u / ng, gi = u - r * ng;
    const int64_t c0 = gi * g;
    const int64_t base = r * ldw;
    float m = 0.0f;
    int bad = 0;
    for (int64_t p = lane; p < g / 2; p += 64) {
      const int64_t c = c0 + 2 * p;
      const float v0 = c < k ? load_f32<DT>(w, base + c) : 0.0f;      // :283-290 zero padding
      const float v1 = c + 1 < k ? load_f32<DT>(w, base + c + 1) : 0.0f;
      bad |= !__builtin_isfinite(v0) | !__builtin_isfinite(v1);
      m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fabsf(v0), __builtin_fabsf(v1)));
    }
    m = wave_max(m);                                 // :293
    bad = wave_or(bad);
    if (bad && lane == 0) flag[0] = 1;
    float s32 = m / 7.0f;                            // :294
    s32 = s32 < 1e-8f ? 1e-8f : s32;
    const uint16_t h = f32_to_f16_bits(s32);         // :295, :313
    const float sq = f16_bits_to_f32(h);             // :298
    if (lane == 0) s[r * ng + gi] = h;
    for (int64_t p = lane; p < g / 2; p += 64) {     // :299-309
      const int64_t c = c0 + 2 * p;
      const float v0 = c < k ? load_f32<DT>(w, base + c) : 0.0f;
      const float v1 = c + 1 < k ? load_f32<DT>(w, base + c + 1) : 0.0f;
      const uint32_t lo = (uint32_t)round_clamp(v0 / sq, -8.0f, 7.0f) & 0xFu;
      const uint32_t hi = (uint32_t)round_clamp(v1 / sq, -8.0f, 7.0f) & 0xFu;
      q[r * row_bytes + c0 / 2 + p] = (uint8_t)(lo | (hi << 4));
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void finite_kernel(const void* __restrict__ w, int64_t n,
                                                     int64_t k, int64_t ldw,
                                                     int32_t* __restrict__ flag) {
  const int64_t total = n * k;
  int bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / k, c = i - r * k;
    bad |= !__builtin_isfinite(load_f32<DT>(w, r * ldw + c));
  }
  bad = wave_or(bad);
  if (bad && (threadIdx.x & 63) == 0) flag[0] = 1;
}

__global__ void zero_flag_kernel(int32_t* flag) { flag[0] = 0; }

template <int ODT>
__device__ __forceinline__ void store_out(void* out, int64_t i, float v) {
  if constexpr (ODT == KQ_F32) static_cast<float*>(out)[i] = v;
  else if constexpr (ODT == KQ_F16) static_cast<uint16_t*>(out)[i] = f32_to_f16_bits(v);
  else static_cast<uint16_t*>(out)[i] = f32_to_bf16_bits_rne(v);
}

template <int ODT>
__global__ __launch_bounds__(256) void dq8_kernel(const int8_t* __restrict__ q,
                                                  const uint16_t* __restrict__ s, int64_t n,
                                                  int64_t k, void* __restrict__ out) {
  const int64_t total = n * k;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / k;
    store_out<ODT>(out, i, (float)q[i] * f16_bits_to_f32(s[r]));   // :228-229
  }
}

template <int ODT>
__global__ __launch_bounds__(256) void dq4_kernel(const uint8_t* __restrict__ q,
                                                  const uint16_t* __restrict__ s, int64_t n,
                                                  int64_t k, int64_t g, int64_t kp,
                                                  void* __restrict__ out) {
  const int64_t total = n * k, ng = kp / g;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / k, c = i - r * k;
    const uint32_t b = q[r * (kp / 2) + (c >> 1)];
    const int u = (c & 1) ? (int)((b >> 4) & 0xFu) : (int)(b & 0xFu);   // :328-333
    const int v = u >= 8 ? u - 16 : u;                                  // :335
    store_out<ODT>(out, i, (float)v * f16_bits_to_f32(s[r * ng + c / g]));  // :337-344
  }
}

inline unsigned grid_for(int64_t items, int per_block, int64_t cap = 65536) {
  int64_t b = (items + per_block - 1) / per_block;
  if (b < 1) b = 1;
  if (b > cap) b = cap;
  return (unsigned)b;
}

int check_common(const void* w, int dt, int64_t n, int64_t k, int64_t ldw, const void* flag) {
  KQ_REQUIRE(w != nullptr && flag != nullptr, "null pointer argument");
  KQ_REQUIRE(dt == KQ_F32 || dt == KQ_F16 || dt == KQ_BF16, "unsupported weight dtype code");
  KQ_REQUIRE(n > 0 && k > 0, "weight must have non-zero dims");
  KQ_REQUIRE(ldw >= k, "leading dimension smaller than in_features");
  return KQ_OK;
}

}  // namespace

extern "C" int kq_check_finite(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw,
                               int32_t* flag, kq_stream_t stream) {
  if (int st = check_common(w, w_dtype, n, k, ldw, flag)) return st;
  hipStream_t st = kq_stream(stream);
  zero_flag_kernel<<<1, 1, 0, st>>>(flag);
  const unsigned grid = grid_for(n * k, 256, 8192);
  switch (w_dtype) {
    case KQ_F32: finite_kernel<KQ_F32><<<grid, 256, 0, st>>>(w, n, k, ldw, flag); break;
    case KQ_F16: finite_kernel<KQ_F16><<<grid, 256, 0, st>>>(w, n, k, ldw, flag); break;
    default: finite_kernel<KQ_BF16><<<grid, 256, 0, st>>>(w, n, k, ldw, flag); break;
  }
  return kq_check_launch("kq_check_finite");
}

extern "C" int kq_quantize_int8(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw,
                                int8_t* payload, uint16_t* scales, int32_t* flag,
                                kq_stream_t stream) {
  if (int st = check_common(w, w_dtype, n, k, ldw, flag)) return st;
  KQ_REQUIRE(payload != nullptr && scales != nullptr, "null output pointer");
  hipStream_t st = kq_stream(stream);
  zero_flag_kernel<<<1, 1, 0, st>>>(flag);
  const unsigned grid = grid_for(n, 1, 65536);
  switch (w_dtype) {
    case KQ_F32: q8_rows_kernel<KQ_F32><<<grid, kQ8Threads, 0, st>>>(w, n, k, ldw, payload, scales, flag); break;
    case KQ_F16: q8_rows_kernel<KQ_F16><<<grid, kQ8Threads, 0, st>>>(w, n, k, ldw, payload, scales, flag); break;
    default: q8_rows_kernel<KQ_BF16><<<grid, kQ8Threads, 0, st>>>(w, n, k, ldw, payload, scales, flag); break;
  }
  return kq_check_launch("kq_quantize_int8");
}

extern "C" int kq_quantize_int4(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw,
                                int64_t g, uint8_t* payload, uint16_t* scales, int32_t* flag,
                                kq_stream_t stream) {
  if (int st = check_common(w, w_dtype, n, k, ldw, flag)) return st;
  KQ_REQUIRE(g > 0 && g % 2 == 0, "group_size must be a positive even integer");
  KQ_REQUIRE(payload != nullptr && scales != nullptr, "null output pointer");
  const int64_t ng = (k + g - 1) / g;
  hipStream_t st = kq_stream(stream);
  zero_flag_kernel<<<1, 1, 0, st>>>(flag);
  const unsigned grid = grid_for(n * ng, 4, 65536);
  switch (w_dtype) {
    case KQ_F32: q4_groups_kernel<KQ_F32><<<grid, 256, 0, st>>>(w, n, k, ldw, g, ng, payload, scales, flag); break;
    case KQ_F16: q4_groups_kernel<KQ_F16><<<grid, 256, 0, st>>>(w, n, k, ldw, g, ng, payload, scales, flag); break;
    default: q4_groups_kernel<KQ_BF16><<<grid, 256, 0, st>>>(w, n, k, ldw, g, ng, payload, scales, flag); break;
  }
  return kq_check_launch("kq_quantize_int4");
}

extern "C" int kq_dequantize_int8(const int8_t* payload, const uint16_t* scales, int64_t n,
                                  int64_t k, void* out, int out_dtype, kq_stream_t stream) {
  KQ_REQUIRE(payload != nullptr && scales != nullptr && out != nullptr, "null pointer argument");
  KQ_REQUIRE(n > 0 && k > 0, "empty weight");
  hipStream_t st = kq_stream(stream);
  const unsigned grid = grid_for(n * k, 256);
  switch (out_dtype) {
    case KQ_F32: dq8_kernel<KQ_F32><<<grid, 256, 0, st>>>(payload, scales, n, k, out); break;
    case KQ_F16: dq8_kernel<KQ_F16><<<grid, 256, 0, st>>>(payload, scales, n, k, out); break;
    case KQ_BF16: dq8_kernel<KQ_BF16><<<grid, 256, 0, st>>>(payload, scales, n, k, out); break;
    default: return kq_set_error(KQ_ERR_ARG, "unsupported output dtype code");
  }
  return kq_check_launch("kq_dequantize_int8");
}

extern "C" int kq_dequantize_int4(const uint8_t* payload, const uint16_t* scales, int64_t n,
                                  int64_t k, int64_t g, int64_t kp, void* out, int out_dtype,
                                  kq_stream_t stream) {
  KQ_REQUIRE(payload != nullptr && scales != nullptr && out != nullptr, "null pointer argument");
  KQ_REQUIRE(n > 0 && k > 0, "empty weight");
  KQ_REQUIRE(g > 0 && g % 2 == 0 && kp % g == 0 && kp >= k && kp - k < g,
             "inconsistent group_size / in_features_padded");
  hipStream_t st = kq_stream(stream);
  const unsigned grid = grid_for(n * k, 256);
  switch (out_dtype) {
    case KQ_F32: dq4_kernel<KQ_F32><<<grid, 256, 0, st>>>(payload, scales, n, k, g, kp, out); break;
    case KQ_F16: dq4_kernel<KQ_F16><<<grid, 256, 0, st>>>(payload, scales, n, k, g, kp, out); break;
    case KQ_BF16: dq4_kernel<KQ_BF16><<<grid, 256, 0, st>>>(payload, scales, n, k, g, kp, out); break;
    default: return kq_set_error(KQ_ERR_ARG, "unsupported output dtype code");
  }
  return kq_check_launch("kq_dequantize_int4");
}
