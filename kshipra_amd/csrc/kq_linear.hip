// Fused dequant-matmul kernels for QuantizedLinear.forward (Kshipra
// engine/quantization.py:394-396): y = x @ (q * s)^T + b, fp32 in/out.
//
// The reference materialises the fp32 weight and calls F.linear.  Here the
// packed payload streams from HBM once and is dequantized in registers:
//
//  * skinny_kernel  (M <= 16, decode): one wavefront owns 16 output columns
//    and a K-slice; each lane issues 16-byte loads of its row (4 lanes cover a
//    64-byte INT4 group / INT8 window), unpacks nibbles or bytes to exact fp16
//    in registers and feeds v_mfma_f32_16x16x32_f16 twice (activation hi and
//    lo halves, fp32 accumulation).  INT4 group scales scale each group's
//    partial sum; INT8 row scales scale the final sum.  The waves of a
//    workgroup split K and are reduced through LDS in a fixed order
//    (deterministic).  The activations are staged as fp16 hi/lo MFMA operands
//    in LDS by the workgroup itself when they fit, else by stage_x_kernel into
//    the caller's workspace.
//  * gemm_kernel    (M > 16, prefill chunks / batched decode): workgroup tile
//    BM x BN; the activation tile of each 128-column stage is copied into LDS
//    and shared by the waves, each wave streams its own weight columns from
//    HBM into registers.
//  * generic_kernel (any group size / K): scalar dequant + FMA fallback for
//    shapes the MFMA paths do not tile.
#include <algorithm>

#include "kq_common.hpp"

namespace {

// ---------------------------------------------------------------------------
// Activation staging.  Entry (T, qd, m) = the 8 fp16 hi and 8 fp16 lo halves
// that lane (qd, m) feeds to k-step T.  Two layouts:
//   kLaneMajor  e = (qd * mrows + m) * pitch + T   (skinny kernel: a lane's
//               k-steps are 16 bytes apart, so one base address serves all)
//   kStepMajor  e = (T * 4 + qd) * mrows + m       (gemm kernel: a stage's
//               entries for a row block are contiguous)
// ---------------------------------------------------------------------------
enum StageLayout { kLaneMajor = 0, kStepMajor = 1 };

template <int BITS>
__device__ __forceinline__ void stage_entry(const float* __restrict__ x, int64_t ldx, int64_t M,
                                            int64_t K, int T, int qd, int64_t m,
                                            half8_t& hi, half8_t& lo) {
  float v[8];
  const int64_t c0 = kstep_col0<BITS>(T, qd);
  if (m < M) {
    const float* row = x + m * ldx;
#pragma unroll
    for (int s = 0; s < 8; s++) {
      const int64_t col = c0 + kstep_perm<BITS>(s);
      v[s] = col < K ? row[col] : 0.0f;
    }
  } else {
#pragma unroll
    for (int s = 0; s < 8; s++) v[s] = 0.0f;
  }
  split_hi_lo(v, hi, lo);
}

// Decompose a dense entry counter into (T, qd, m) and the layout's index.
template <int LAYOUT>
__device__ __forceinline__ int64_t stage_index(int64_t e, int64_t nT, int64_t mrows, int64_t pitch,
                                               int& T, int& qd, int64_t& m) {
  if constexpr (LAYOUT == kLaneMajor) {
    T = (int)(e % nT);
    const int64_t r = e / nT;
    m = r % mrows;
    qd = (int)(r / mrows);
    return (qd * mrows + m) * pitch + T;
  } else {
    m = e % mrows;
    const int64_t t = e / mrows;
    qd = (int)(t & 3);
    T = (int)(t >> 2);
    return e;
  }
}

template <int BITS, int LAYOUT>
__global__ __launch_bounds__(256) void stage_x_kernel(const float* __restrict__ x, int64_t ldx,
                                                      int64_t M, int64_t K, int64_t nT,
                                                      int64_t mrows, int64_t pitch,
                                                      half8_t* __restrict__ xa_hi,
                                                      half8_t* __restrict__ xa_lo) {
  const int64_t total = nT * 4 * mrows;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int T, qd;
    int64_t m;
    const int64_t idx = stage_index<LAYOUT>(e, nT, mrows, pitch, T, qd, m);
    half8_t hi, lo;
    stage_entry<BITS>(x, ldx, M, K, T, qd, m, hi, lo);
    xa_hi[idx] = hi;
    xa_lo[idx] = lo;
  }
}

// ---------------------------------------------------------------------------
// Skinny kernel: M <= 16.  grid.x = ceil(N / 16) column tiles; blockDim =
// 64 * W, wave w owns units [w * per_wave, (w + 1) * per_wave) (unit = INT4
// group of 128 columns / INT8 window of 64 columns), loaded KS at a time.
// ---------------------------------------------------------------------------
template <int BITS, int KS, bool A_LDS>
__global__ __launch_bounds__(1024) void skinny_kernel(
    const float* __restrict__ x, int64_t ldx, int M, int64_t K,
    const uint8_t* __restrict__ wq, const uint16_t* __restrict__ sc, int64_t row_bytes,
    int64_t ng, int64_t nunits, int64_t per_wave, int pitch, const half8_t* __restrict__ xa_hi,
    const half8_t* __restrict__ xa_lo, const float* __restrict__ bias, float* __restrict__ y,
    int64_t ldy, int64_t N) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int TPU = BITS == 4 ? 4 : 2;  // k-steps per unit
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int qd = lane >> 4, c = lane & 15;
  const int nT = (int)(nunits * TPU);

  const half8_t* a_hi = xa_hi;
  const half8_t* a_lo = xa_lo;
  if constexpr (A_LDS) {
    half8_t* l_hi = reinterpret_cast<half8_t*>(smem);
    half8_t* l_lo = l_hi + 4 * M * pitch;
    const int entries = nT * 4 * M;
    for (int e = tid; e < entries; e += blockDim.x) {
      int T, q4;
      int64_t m;
      const int idx = (int)stage_index<kLaneMajor>(e, nT, M, pitch, T, q4, m);
      half8_t hi, lo;
      stage_entry<BITS>(x, ldx, M, K, T, q4, m, hi, lo);
      l_hi[idx] = hi;
      l_lo[idx] = lo;
    }
    __syncthreads();
    a_hi = l_hi;
    a_lo = l_lo;
  }
  // This lane's activation entries: k-step T at a_*_lane[T].
  const int a_row = c < M ? c : 0;
  const half8_t* a_hi_lane = a_hi + (int64_t)(qd * M + a_row) * pitch;
  const half8_t* a_lo_lane = a_lo + (int64_t)(qd * M + a_row) * pitch;

  const int64_t n = (int64_t)blockIdx.x * 16 + c;
  const int64_t nl = n < N ? n : N - 1;
  const uint8_t* wrow = wq + nl * row_bytes + qd * 16;
  const int64_t ub = (int64_t)wave * per_wave;
  const int64_t ue = ub + per_wave < nunits ? ub + per_wave : nunits;
  const bool a_lane = c < M;  // lanes holding activation row c; the rest stay zero

  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  half8_t ah[TPU], al[TPU];
#pragma unroll
  for (int i = 0; i < TPU; i++) { ah[i] = half8_t{}; al[i] = half8_t{}; }

  for (int64_t u0 = ub; u0 < ue; u0 += KS) {
    u32x4 raw[KS];
#pragma unroll
    for (int u = 0; u < KS; u++) {
      const int64_t unit = u0 + u < ue ? u0 + u : ue - 1;  // tail: reload the last unit, unused
      raw[u] = *reinterpret_cast<const u32x4*>(wrow + unit * 64);
    }
#pragma unroll
    for (int u = 0; u < KS; u++) {
      if (u0 + u < ue) {
        const int64_t unit = u0 + u;
        if (a_lane) {
#pragma unroll
          for (int i = 0; i < TPU; i++) {
            ah[i] = a_hi_lane[unit * TPU + i];
            al[i] = a_lo_lane[unit * TPU + i];
          }
        }
        if constexpr (BITS == 4) {
          const float s = f16_bits_to_f32(sc[nl * ng + unit]);
          floatx4 g = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const half8_t b = int4x8_to_half8(raw[u][i]);
            g = mfma16x16x32(ah[i], b, g);
            g = mfma16x16x32(al[i], b, g);
          }
#pragma unroll
          for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(s, g[i], acc[i]);
        } else {
#pragma unroll
          for (int j = 0; j < 2; j++) {
            const half8_t b = int8x8_to_half8(raw[u][2 * j], raw[u][2 * j + 1]);
            acc = mfma16x16x32(ah[j], b, acc);
            acc = mfma16x16x32(al[j], b, acc);
          }
        }
      }
      // Keep each unit's operand loads and conversions next to its MFMAs;
      // hoisting every unit's operands above the first one exhausts VGPRs.
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Cross-wave reduction in a fixed order.  Lane (qd, c) holds rows 4qd+i, column c.
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < 4; i++) red[(wave * 16 + 4 * qd + i) * 16 + c] = acc[i];
  __syncthreads();
  for (int o = tid; o < M * 16; o += blockDim.x) {
    const int m = o >> 4, cc = o & 15;
    const int64_t nn = (int64_t)blockIdx.x * 16 + cc;
    if (nn < N) {
      float v = 0.0f;
      for (int w = 0; w < nwaves; w++) v += red[(w * 16 + m) * 16 + cc];
      if constexpr (BITS == 8) v *= f16_bits_to_f32(sc[nn]);
      if (bias) v += bias[nn];
      y[m * ldy + nn] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// GEMM kernel: M > 16.  Workgroup = WN waves along N; tile BM = 16 * MTW rows
// by BN = 16 * NTW * WN columns; one stage = 128 columns of K (4 k-steps).
// Activation entries come from the staged workspace (mrows = M rounded up to
// BM, zero rows past M).
// ---------------------------------------------------------------------------
template <int BITS, int MTW, int NTW, int WN>
__global__ __launch_bounds__(64 * WN) void gemm_kernel(
    const half8_t* __restrict__ xa_hi, const half8_t* __restrict__ xa_lo, int64_t mrows,
    const uint8_t* __restrict__ wq, const uint16_t* __restrict__ sc, int64_t row_bytes,
    int64_t ng, int64_t nstages, const float* __restrict__ bias, float* __restrict__ y,
    int64_t ldy, int64_t M, int64_t N) {
  constexpr int BM = 16 * MTW;
  constexpr int ENTRIES = 16 * BM;  // 4 k-steps x 4 quads x BM rows per stage
  constexpr int RAWN = BITS == 4 ? 1 : 2;
  __shared__ half8_t l_hi[ENTRIES];
  __shared__ half8_t l_lo[ENTRIES];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qd = lane >> 4, c = lane & 15;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = ((int64_t)blockIdx.x * WN + wave) * (16 * NTW);

  const uint8_t* wrow[NTW];
  int64_t nrow[NTW];
#pragma unroll
  for (int t = 0; t < NTW; t++) {
    const int64_t n = n0 + t * 16 + c;
    nrow[t] = n < N ? n : N - 1;
    wrow[t] = wq + nrow[t] * row_bytes + qd * 16;
  }

  floatx4 acc[MTW][NTW];
  floatx4 gacc[MTW][NTW];
#pragma unroll
  for (int i = 0; i < MTW; i++)
#pragma unroll
    for (int t = 0; t < NTW; t++) {
      acc[i][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      gacc[i][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }

  for (int64_t st = 0; st < nstages; st++) {
    u32x4 raw[NTW][RAWN];
#pragma unroll
    for (int t = 0; t < NTW; t++)
#pragma unroll
      for (int r = 0; r < RAWN; r++)
        raw[t][r] = *reinterpret_cast<const u32x4*>(wrow[t] + (st * RAWN + r) * 64);

    __syncthreads();
    for (int e = tid; e < ENTRIES; e += 64 * WN) {
      const int mm = e % BM, tq = e / BM;  // tq = local T * 4 + qd
      const int64_t ge = ((st * 4 + (tq >> 2)) * 4 + (tq & 3)) * mrows + m0 + mm;
      l_hi[e] = xa_hi[ge];
      l_lo[e] = xa_lo[ge];
    }
    __syncthreads();

#pragma unroll
    for (int i = 0; i < 4; i++) {
      half8_t b[NTW];
#pragma unroll
      for (int t = 0; t < NTW; t++) {
        if constexpr (BITS == 4) b[t] = int4x8_to_half8(raw[t][0][i]);
        else b[t] = int8x8_to_half8(raw[t][i >> 1][2 * (i & 1)], raw[t][i >> 1][2 * (i & 1) + 1]);
      }
#pragma unroll
      for (int mt = 0; mt < MTW; mt++) {
        const int e = (i * 4 + qd) * BM + mt * 16 + c;
        const half8_t ah = l_hi[e], al = l_lo[e];
#pragma unroll
        for (int t = 0; t < NTW; t++) {
          gacc[mt][t] = mfma16x16x32(ah, b[t], gacc[mt][t]);
          gacc[mt][t] = mfma16x16x32(al, b[t], gacc[mt][t]);
        }
      }
    }
    if constexpr (BITS == 4) {
#pragma unroll
      for (int t = 0; t < NTW; t++) {
        const float s = f16_bits_to_f32(sc[nrow[t] * ng + st]);
#pragma unroll
        for (int mt = 0; mt < MTW; mt++) {
#pragma unroll
          for (int i = 0; i < 4; i++) acc[mt][t][i] = __builtin_fmaf(s, gacc[mt][t][i], acc[mt][t][i]);
          gacc[mt][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
    }
  }

#pragma unroll
  for (int t = 0; t < NTW; t++) {
    const int64_t n = n0 + t * 16 + c;
    if (n >= N) continue;
    float s8 = 1.0f;
    if constexpr (BITS == 8) s8 = f16_bits_to_f32(sc[n]);
    const float b = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MTW; mt++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + mt * 16 + 4 * qd + i;
        if (m < M) {
          const float v = BITS == 4 ? acc[mt][t][i] : gacc[mt][t][i] * s8;
          y[m * ldy + n] = v + b;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Generic fallback: any K, any even group size.  One wavefront per output
// column n, four activation rows at a time, fp32 FMA of the exact dequantized
// weight.
// ---------------------------------------------------------------------------
template <int BITS>
__global__ __launch_bounds__(256) void generic_kernel(const float* __restrict__ x, int64_t ldx,
                                                      int64_t M, const uint8_t* __restrict__ wq,
                                                      const uint16_t* __restrict__ sc,
                                                      int64_t row_bytes, int64_t g, int64_t ng,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int64_t ldy,
                                                      int64_t N, int64_t K) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t n = wave0; n < N; n += wstride) {
    const uint8_t* row = wq + n * row_bytes;
    for (int64_t m0 = 0; m0 < M; m0 += 4) {
      float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int64_t k = lane; k < K; k += 64) {
        float wv;
        if constexpr (BITS == 8) {
          wv = (float)(int8_t)row[k] * f16_bits_to_f32(sc[n]);
        } else {
          const uint32_t b = row[k >> 1];
          const int u = (k & 1) ? (int)((b >> 4) & 0xFu) : (int)(b & 0xFu);
          wv = (float)(u >= 8 ? u - 16 : u) * f16_bits_to_f32(sc[n * ng + k / g]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
          if (m0 + j < M) a[j] = __builtin_fmaf(x[(m0 + j) * ldx + k], wv, a[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float v = wave_sum(a[j]);
        if (lane == 0 && m0 + j < M) y[(m0 + j) * ldy + n] = v + (bias ? bias[n] : 0.0f);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
constexpr int kSkinnyMaxM = 16;
constexpr int kSkinnyMaxWaves = 16;
constexpr int64_t kSkinnyLdsA = 64 * 1024;  // activation bytes staged in LDS by the workgroup
constexpr int kGemmMTW = 4, kGemmNTW = 4, kGemmWN = 4;
constexpr int64_t kGemmBM = 16 * kGemmMTW;
constexpr int64_t kGemmBN = 16 * kGemmNTW * kGemmWN;

enum class Path { Skinny, Gemm, Generic };

struct Plan {
  Path path;
  int ks = 0;           // skinny: units per wave
  int waves = 0;        // skinny: waves per workgroup
  int64_t per_wave = 0; // skinny: units per wave (processed KS at a time)
  bool a_lds = false;   // skinny: activations staged in LDS
  int64_t nunits = 0;   // INT4 groups / INT8 windows per row
  int64_t nT = 0;       // k-steps
  int64_t mrows = 0;    // staged activation rows
  int64_t pitch = 0;    // skinny: entries per (quad, row) in the lane-major layout
  size_t ws = 0;        // workspace bytes
};

Plan make_plan(int bits, int64_t m, int64_t n, int64_t k, int64_t g, int64_t kp) {
  Plan p;
  const bool tiled = bits == 4 ? (g == 128) : (k % 64 == 0);
  if (!tiled) { p.path = Path::Generic; return p; }
  p.nunits = bits == 4 ? kp / 128 : k / 64;
  p.nT = p.nunits * (bits == 4 ? 4 : 2);
  if (m <= kSkinnyMaxM) {
    int ks = 4;
    while (ks < 16 && (p.nunits + ks - 1) / ks > kSkinnyMaxWaves) ks *= 2;
    p.path = Path::Skinny;
    p.ks = ks;
    p.waves = (int)std::min<int64_t>((p.nunits + ks - 1) / ks, kSkinnyMaxWaves);
    p.per_wave = (p.nunits + p.waves - 1) / p.waves;
    p.mrows = m;
    // An odd pitch puts the four lane quads of an LDS row in different banks.
    p.pitch = p.nT | 1;
    p.a_lds = 128 * p.pitch * m <= kSkinnyLdsA;  // 2 planes x 16 B x 4 quads per entry
    if (!p.a_lds) p.pitch = p.nT;
    p.ws = p.a_lds ? 0 : (size_t)(128 * p.pitch * m);
    return p;
  }
  const int64_t keff = p.nT * 32;
  if (keff % 128 != 0) { p.path = Path::Generic; return p; }
  p.path = Path::Gemm;
  p.mrows = (m + kGemmBM - 1) / kGemmBM * kGemmBM;
  p.ws = (size_t)(4 * keff * p.mrows);
  (void)n;
  return p;
}

template <int BITS>
int launch_skinny(const Plan& p, const float* x, int64_t ldx, int64_t m, int64_t k,
                  const uint8_t* wq, const uint16_t* sc, int64_t row_bytes, int64_t ng,
                  const float* bias, float* y, int64_t ldy, int64_t n, void* ws, hipStream_t st) {
  const half8_t* xh = nullptr;
  const half8_t* xl = nullptr;
  if (!p.a_lds) {
    half8_t* h = static_cast<half8_t*>(ws);
    half8_t* l = h + p.pitch * 4 * m;  // planes of 4 * m * pitch entries
    const int64_t entries = p.nT * 4 * m;
    unsigned grid = (unsigned)std::min<int64_t>((entries + 255) / 256, 4096);
    stage_x_kernel<BITS, kLaneMajor><<<grid, 256, 0, st>>>(x, ldx, m, k, p.nT, m, p.pitch, h, l);
    xh = h;
    xl = l;
  }
  const size_t red = (size_t)p.waves * 256 * sizeof(float);
  const size_t a = p.a_lds ? (size_t)(4 * p.pitch * 32 * m) : 0;
  const size_t shm = std::max(red, a);
  const dim3 grid((unsigned)((n + 15) / 16));
  const dim3 block((unsigned)(64 * p.waves));
#define KQ_SKINNY(KS_, LDS_)                                                                  \
  skinny_kernel<BITS, KS_, LDS_><<<grid, block, shm, st>>>(x, ldx, (int)m, k, wq, sc,       \
                                                           row_bytes, ng, p.nunits,         \
                                                           p.per_wave, (int)p.pitch, xh, xl, \
                                                           bias, y, ldy, n)
  if (p.a_lds) {
    switch (p.ks) {
      case 4: KQ_SKINNY(4, true); break;
      case 8: KQ_SKINNY(8, true); break;
      default: KQ_SKINNY(16, true); break;
    }
  } else {
    switch (p.ks) {
      case 4: KQ_SKINNY(4, false); break;
      case 8: KQ_SKINNY(8, false); break;
      default: KQ_SKINNY(16, false); break;
    }
  }
#undef KQ_SKINNY
  return kq_check_launch(BITS == 4 ? "kq_linear_int4 (skinny)" : "kq_linear_int8 (skinny)");
}

template <int BITS>
int launch_gemm(const Plan& p, const float* x, int64_t ldx, int64_t m, int64_t k,
                const uint8_t* wq, const uint16_t* sc, int64_t row_bytes, int64_t ng,
                const float* bias, float* y, int64_t ldy, int64_t n, void* ws, hipStream_t st) {
  half8_t* h = static_cast<half8_t*>(ws);
  half8_t* l = h + p.nT * 4 * p.mrows;
  const int64_t entries = p.nT * 4 * p.mrows;
  unsigned sgrid = (unsigned)std::min<int64_t>((entries + 255) / 256, 8192);
  stage_x_kernel<BITS, kStepMajor><<<sgrid, 256, 0, st>>>(x, ldx, m, k, p.nT, p.mrows, 0, h, l);
  const dim3 grid((unsigned)((n + kGemmBN - 1) / kGemmBN), (unsigned)(p.mrows / kGemmBM));
  gemm_kernel<BITS, kGemmMTW, kGemmNTW, kGemmWN><<<grid, 64 * kGemmWN, 0, st>>>(
      h, l, p.mrows, wq, sc, row_bytes, ng, p.nT / 4, bias, y, ldy, m, n);
  return kq_check_launch(BITS == 4 ? "kq_linear_int4 (gemm)" : "kq_linear_int8 (gemm)");
}

template <int BITS>
int launch_generic(const float* x, int64_t ldx, int64_t m, const uint8_t* wq, const uint16_t* sc,
                   int64_t row_bytes, int64_t g, int64_t ng, const float* bias, float* y,
                   int64_t ldy, int64_t n, int64_t k, hipStream_t st) {
  unsigned grid = (unsigned)std::min<int64_t>((n + 3) / 4, 65536);
  generic_kernel<BITS><<<grid, 256, 0, st>>>(x, ldx, m, wq, sc, row_bytes, g, ng, bias, y, ldy, n, k);
  return kq_check_launch(BITS == 4 ? "kq_linear_int4 (generic)" : "kq_linear_int8 (generic)");
}

int check_linear_args(const float* x, int64_t m, int64_t ldx, const void* wq, const void* sc,
                      float* y, int64_t ldy, int64_t n, int64_t k) {
  KQ_REQUIRE(x != nullptr && wq != nullptr && sc != nullptr && y != nullptr, "null pointer argument");
  KQ_REQUIRE(m > 0 && n > 0 && k > 0, "empty linear");
  KQ_REQUIRE(ldx >= k, "ldx smaller than in_features");
  KQ_REQUIRE(ldy >= n, "ldy smaller than out_features");
  return KQ_OK;
}

}  // namespace

extern "C" size_t kq_linear_workspace_bytes(int scheme, int64_t m, int64_t n, int64_t k,
                                            int64_t group_size) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  if (scheme == 8) return make_plan(8, m, n, k, 0, k).ws;
  if (group_size <= 0) return 0;
  const int64_t kp = (k + group_size - 1) / group_size * group_size;
  return make_plan(4, m, n, k, group_size, kp).ws;
}

extern "C" int kq_linear_int8(const float* x, int64_t m, int64_t ldx, const int8_t* payload,
                              const uint16_t* scales, const float* bias, float* y, int64_t ldy,
                              int64_t n, int64_t k, void* ws, size_t ws_bytes,
                              kq_stream_t stream) {
  if (int s = check_linear_args(x, m, ldx, payload, scales, y, ldy, n, k)) return s;
  const Plan p = make_plan(8, m, n, k, 0, k);
  if (p.ws > 0 && (ws == nullptr || ws_bytes < p.ws))
    return kq_set_error(KQ_ERR_WORKSPACE, "workspace missing or smaller than kq_linear_workspace_bytes()");
  const uint8_t* wq = reinterpret_cast<const uint8_t*>(payload);
  hipStream_t st = kq_stream(stream);
  switch (p.path) {
    case Path::Skinny: return launch_skinny<8>(p, x, ldx, m, k, wq, scales, k, 1, bias, y, ldy, n, ws, st);
    case Path::Gemm: return launch_gemm<8>(p, x, ldx, m, k, wq, scales, k, 1, bias, y, ldy, n, ws, st);
    default: return launch_generic<8>(x, ldx, m, wq, scales, k, 1, 1, bias, y, ldy, n, k, st);
  }
}

extern "C" int kq_linear_int4(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                              const uint16_t* scales, int64_t g, int64_t kp, const float* bias,
                              float* y, int64_t ldy, int64_t n, int64_t k, void* ws,
                              size_t ws_bytes, kq_stream_t stream) {
  if (int s = check_linear_args(x, m, ldx, payload, scales, y, ldy, n, k)) return s;
  KQ_REQUIRE(g > 0 && g % 2 == 0, "group_size must be a positive even integer");
  KQ_REQUIRE(kp % g == 0 && kp >= k && kp - k < g, "inconsistent in_features_padded");
  const Plan p = make_plan(4, m, n, k, g, kp);
  if (p.ws > 0 && (ws == nullptr || ws_bytes < p.ws))
    return kq_set_error(KQ_ERR_WORKSPACE, "workspace missing or smaller than kq_linear_workspace_bytes()");
  const int64_t ng = kp / g;
  hipStream_t st = kq_stream(stream);
  switch (p.path) {
    case Path::Skinny: return launch_skinny<4>(p, x, ldx, m, k, payload, scales, kp / 2, ng, bias, y, ldy, n, ws, st);
    case Path::Gemm: return launch_gemm<4>(p, x, ldx, m, k, payload, scales, kp / 2, ng, bias, y, ldy, n, ws, st);
    default: return launch_generic<4>(x, ldx, m, payload, scales, kp / 2, g, ng, bias, y, ldy, n, k, st);
  }
}
