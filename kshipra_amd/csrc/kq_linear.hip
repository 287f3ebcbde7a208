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
//    in LDS by the workgroup itself when they fit (each wave scales its own
//    K-slice of a row), else by stage_rows_kernel into the caller's
//    workspace (one scale per row).
//  * gemm_kernel    (17 <= M <= 32, batched decode): workgroup tile BM x 128
//    (x 256 for very wide N); x is converted once per call into fp16 hi/lo operand planes
//    (stage_rows_kernel), each 128-column stage of them is copied into LDS
//    (double-buffered) and shared by the waves; each wave streams its own
//    weight columns from HBM into registers one stage ahead.  K is split across workgroups when the tiles alone cannot
//    fill the GPU; partials are then added in a fixed order.
//  * gemm_ws_kernel (prefill chunks): warp-specialised variant fed by DMA.
//  * generic_kernel (any group size / K): scalar dequant + FMA fallback for
//    shapes the MFMA paths do not tile.
#include <algorithm>

#include "kq_common.hpp"

namespace {

// ---------------------------------------------------------------------------
// Activation staging.  An "entry" (T, qd, m) is the 8 activations of row m that
// lane quad qd feeds to k-step T, scaled by the power of two 2^e of its row
// (or row-slice; kq_common.hpp) and split into fp16 hi and lo halves.  Every
// sum over staged entries is scaled back by 2^-e before it leaves the
// kernel (partials included).
//
// Skinny layout (lane-major, one array): A-row r, quad qd, k-step T at
//   index (qd * R + r) * pitch + T,   a lane's k-steps 16 bytes apart.
//   HL mode (M <= 8): R = 2M rows; row m = hi(x[m]), row M + m = lo(x[m]).
//     The MFMA sees hi and lo as different A rows, so one MFMA per k-step
//     yields both partial sums (rows m and m + 8 of the output tile).
//   split mode (M <= 16): R = M rows in two arrays (hi, lo); two MFMAs per k-step.
// GEMM operand planes: see stage_rows_kernel.
// ---------------------------------------------------------------------------
// Load the 8 consecutive activations of entry (T, qd, m) (zeros past M / K).
template <int BITS>
__device__ __forceinline__ void stage_load(const float* __restrict__ x, int64_t ldx, int64_t M,
                                           int64_t K, int T, int qd, int64_t m, bool xvec,
                                           float (&raw8)[8]) {
  const int64_t c0 = kstep_col0<BITS>(T, qd);
  if (m < M) {
    const float* src = x + m * ldx + c0;
    if (xvec && c0 + 8 <= K) {
      const float4 a = reinterpret_cast<const float4*>(src)[0];
      const float4 b = reinterpret_cast<const float4*>(src)[1];
      raw8[0] = a.x; raw8[1] = a.y; raw8[2] = a.z; raw8[3] = a.w;
      raw8[4] = b.x; raw8[5] = b.y; raw8[6] = b.z; raw8[7] = b.w;
    } else {
#pragma unroll
      for (int s = 0; s < 8; s++) raw8[s] = c0 + s < K ? src[s] : 0.0f;
    }
  } else {
#pragma unroll
    for (int s = 0; s < 8; s++) raw8[s] = 0.0f;
  }
}

// Permute the 8 loaded activations into operand-slot order, scale them by
// 2^e and split them (guard: wave_has_inf of the converting lanes' maxima).
template <int BITS>
__device__ __forceinline__ void stage_convert(const float (&raw8)[8], int e, half8_t& hi, half8_t& lo,
                                              bool guard) {
  float v[8];
#pragma unroll
  for (int s = 0; s < 8; s++) v[s] = raw8[kstep_perm<BITS>(s)];
  split_hi_lo(v, e, hi, lo, guard);
}

// Skinny layout: the two 16-byte slots of entry (T, qd, m).  HL: one array,
// rows m and M + m; split: the hi array, then the lo array.
template <bool HL>
__device__ __forceinline__ void skinny_slots(int M, int64_t pitch, int T, int qd, int m,
                                             int64_t& ihi, int64_t& ilo) {
  if constexpr (HL) {
    ihi = (int64_t)(qd * 2 * M + m) * pitch + T;
    ilo = (int64_t)(qd * 2 * M + M + m) * pitch + T;
  } else {
    ihi = (int64_t)(qd * M + m) * pitch + T;
    ilo = (int64_t)4 * M * pitch + ihi;
  }
}

template <bool HL>
__device__ __forceinline__ void skinny_store(half8_t* __restrict__ a, int M, int64_t pitch,
                                             int T, int qd, int m, half8_t hi, half8_t lo) {
  int64_t ihi, ilo;
  skinny_slots<HL>(M, pitch, T, qd, m, ihi, ilo);
  a[ihi] = hi;
  a[ilo] = lo;
}

// The raw fp32 values of an entry parked in its own two slots (32 bytes, the
// size of the hi / lo pair) until the slice's scale is known.
template <bool HL>
__device__ __forceinline__ void skinny_park(half8_t* __restrict__ a, int M, int64_t pitch, int T,
                                            int qd, int m, const float (&raw8)[8]) {
  int64_t ihi, ilo;
  skinny_slots<HL>(M, pitch, T, qd, m, ihi, ilo);
  reinterpret_cast<floatx4*>(a)[ihi] = floatx4{raw8[0], raw8[1], raw8[2], raw8[3]};
  reinterpret_cast<floatx4*>(a)[ilo] = floatx4{raw8[4], raw8[5], raw8[6], raw8[7]};
}

template <bool HL>
__device__ __forceinline__ void skinny_unpark(const half8_t* __restrict__ a, int M, int64_t pitch,
                                              int T, int qd, int m, float (&raw8)[8]) {
  int64_t ihi, ilo;
  skinny_slots<HL>(M, pitch, T, qd, m, ihi, ilo);
  const floatx4 u = reinterpret_cast<const floatx4*>(a)[ihi];
  const floatx4 v = reinterpret_cast<const floatx4*>(a)[ilo];
#pragma unroll
  for (int s = 0; s < 4; s++) { raw8[s] = u[s]; raw8[4 + s] = v[s]; }
}

// Largest |x| of the rows a workgroup of 64 * W threads stages (one value per
// thread in, the workgroup maximum out; red holds W floats).
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max_uniform(v);
  const int nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = red[0];
  for (int w = 1; w < nw; w++) v = __builtin_fmaxf(v, red[w]);
  return v;
}

// Stage whole activation rows, one workgroup per row m: the row's scale
// exponent e (written to rexp[m]) from its largest |x|, then every entry
// (T, qd) of the row converted with it.  Rows past M are zeros with e = 0.
//   PLANES = false: skinny layout (HL or split), `pitch` entries per A-row.
//   PLANES = true:  GEMM operand planes: entry (plane p, stage st, row m, e)
//                   at ((p * nstages + st) * Mp + m) * 16 + e, e = (T % 4) * 4 + qd,
//                   st = T / 4 (nT = 4 * nstages, gridDim.x = Mp).
// A thread holds up to kStageHold entries in registers between the maximum
// and the conversion; longer rows are read twice (the second read hits L2).
constexpr int kStageHold = 8;
template <int BITS, bool PLANES, bool HL>
__global__ __launch_bounds__(256) void stage_rows_kernel(const float* __restrict__ x, int64_t ldx,
                                                         int M, int64_t K, int nT, int64_t pitch,
                                                         int64_t Mp, bool xvec,
                                                         half8_t* __restrict__ a,
                                                         int* __restrict__ rexp) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  const int64_t E = (int64_t)nT * 4;
  auto store = [&](int64_t q, half8_t hi, half8_t lo) {
    const int T = (int)(q >> 2), qd = (int)(q & 3);
    if constexpr (PLANES) {
      const int64_t o = ((int64_t)(T >> 2) * Mp + m) * 16 + (T & 3) * 4 + qd;
      const int64_t total = (int64_t)(nT >> 2) * Mp * 16;
      a[o] = hi;
      a[total + o] = lo;
    } else {
      skinny_store<HL>(a, M, pitch, T, qd, m, hi, lo);
    }
  };
  float amax = 0.0f;
  if (E <= (int64_t)kStageHold * blockDim.x) {
    float raw[kStageHold][8];
#pragma unroll
    for (int j = 0; j < kStageHold; j++) {
      const int64_t q = threadIdx.x + (int64_t)j * blockDim.x;
      stage_load<BITS>(x, ldx, M, K, (int)(q >> 2), (int)(q & 3), q < E ? m : M, xvec, raw[j]);
      amax = absmax8(raw[j], amax);
    }
    const int e = act_exponent(block_max(amax, red));
    const bool guard = wave_has_inf(amax);
#pragma unroll
    for (int j = 0; j < kStageHold; j++) {
      const int64_t q = threadIdx.x + (int64_t)j * blockDim.x;
      if (q < E) {
        half8_t hi, lo;
        stage_convert<BITS>(raw[j], e, hi, lo, guard);
        store(q, hi, lo);
      }
    }
    if (threadIdx.x == 0) rexp[m] = e;
  } else {
    for (int64_t q = threadIdx.x; q < E; q += blockDim.x) {
      float raw[8];
      stage_load<BITS>(x, ldx, M, K, (int)(q >> 2), (int)(q & 3), m, xvec, raw);
      amax = absmax8(raw, amax);
    }
    const int e = act_exponent(block_max(amax, red));
    const bool guard = wave_has_inf(amax);
    for (int64_t q = threadIdx.x; q < E; q += blockDim.x) {
      float raw[8];
      stage_load<BITS>(x, ldx, M, K, (int)(q >> 2), (int)(q & 3), m, xvec, raw);
      half8_t hi, lo;
      stage_convert<BITS>(raw, e, hi, lo, guard);
      store(q, hi, lo);
    }
    if (threadIdx.x == 0) rexp[m] = e;
  }
}

// Lanes per activation row in the skinny kernel's in-workgroup staging: 64
// over M rounded up to a power of two (M <= 16: at least 4).
__host__ __device__ inline int skinny_lanes_per_row(int M) {
  int p = 1;
  while (p < M) p <<= 1;
  return 64 / p;
}

// Group scales of units [u0, u0 + KS) of one row.  SVEC: one vector load of
// the KS consecutive fp16 scales (row and u0 aligned to KS), so a wave issues
// one load per row for KS units instead of KS loads; else one load per unit,
// clamped to the last valid unit.
template <int KS, bool SVEC>
__device__ __forceinline__ void load_scales(const uint16_t* __restrict__ srow, int64_t u0,
                                            int64_t ue, uint16_t (&sv)[KS]) {
  if constexpr (SVEC) {
    const uint16_t* p = srow + u0;
    if constexpr (KS == 2) {
      const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
      sv[0] = (uint16_t)v; sv[1] = (uint16_t)(v >> 16);
    } else {
#pragma unroll
      for (int h = 0; h < KS / 8 + (KS < 8); h++) {
        if constexpr (KS == 4) {
          const uint2 v = *reinterpret_cast<const uint2*>(p);
          const uint32_t w[2] = {v.x, v.y};
#pragma unroll
          for (int i = 0; i < 4; i++) sv[i] = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
        } else {
          const u32x4 v = *reinterpret_cast<const u32x4*>(p + 8 * h);
#pragma unroll
          for (int i = 0; i < 8; i++) sv[8 * h + i] = (uint16_t)(v[i >> 1] >> (16 * (i & 1)));
        }
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < KS; u++) sv[u] = srow[u0 + u < ue ? u0 + u : ue - 1];
  }
}

// ---------------------------------------------------------------------------
// Greedy argmax (engine/model.py:187,200: first index of the maximum, as
// torch.argmax): a NaN counts as larger than every number; among equal
// values (+0 == -0) the smaller index wins.  Partials are (value bits, index)
// pairs; index INT32_MAX marks "no column".
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool arg_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

// Reduce a (value, index) pair over the 16 lanes of each 16-lane group.
__device__ __forceinline__ void arg_reduce16(float& v, int& i) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(i, off);
    if (arg_better(ov, oi, v, i)) { v = ov; i = oi; }
  }
}

// ---------------------------------------------------------------------------
// Skinny kernel: M <= 16.  grid.x = ceil(N / (16 * NT)); a workgroup owns NT
// adjacent 16-column tiles and blockDim = 64 * W waves split K: wave w owns
// units [w * per_wave, (w + 1) * per_wave) of every tile (unit = INT4 group
// of 128 columns / INT8 window of 64 columns), loaded KS at a time.  One
// activation operand read feeds the NT tiles' MFMAs, and the workgroup's
// activation staging is shared by 16 * NT columns.  The first chunk's weight
// loads are issued before the activations are staged, so HBM latency
// overlaps the staging.
// ---------------------------------------------------------------------------
// 16 units x tiles per batch need more than the 128 VGPRs a 1024-thread
// workgroup allows: such kernels run at most 8 waves per workgroup (256 VGPRs,
// no spills).
template <int KS, int NT>
constexpr int skinny_max_threads() { return KS * NT >= 16 ? 512 : 1024; }

// M1: instances for M == 1 exactly (one row: pre-load count and layout known
// at compile time, no row stepping).  REM: activation entries may remain after
// the pre-loads (unaligned or K-tail x, more entries than pre-load slots), so
// the code loading them after the weights is compiled in; the host launches
// REM = false instances only when the pre-loads cover every entry (a
// possibly-taken block of loads behind the weights would make the compiler
// wait for all weight loads before the first MFMA).
// wq / sc are deliberately not __restrict__: loads through restrict read-only
// kernel arguments count as invariant and may be sunk past the asm ordering
// fences, which moved the first batch's weight loads behind the staging.
template <int BITS, int KS, int NT, bool A_LDS, bool HL, bool SVEC, bool M1, bool REM>
__global__ __launch_bounds__((skinny_max_threads<KS, NT>())) void skinny_kernel(
    const float* __restrict__ x, int64_t ldx, int M_, int64_t K, bool xvec,
    const uint8_t* wq, const uint16_t* sc, int64_t row_bytes,
    int64_t ng, int64_t nunits, int64_t per_wave, int pitch, const half8_t* __restrict__ xa,
    const int* __restrict__ xexp, const float* __restrict__ bias, float* __restrict__ y,
    int64_t ldy, int64_t N,
    int2* __restrict__ argp, int pairs, int64_t split_units, int64_t split_ystride) {
  static_assert(!M1 || (A_LDS && HL && !REM), "single-row instances stage in LDS, pre-loads only");
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int TPU = BITS == 4 ? 4 : 2;  // k-steps per unit
  const int M = M1 ? 1 : M_;
  // K split across blockIdx.y: workgroup row z owns units [z s, (z + 1) s)
  // (s = split_units) -- its columns of x, payload (64 bytes per unit of a
  // row, both schemes) and INT4 group scales -- and writes its partial sums
  // (row scale applied, no bias) to y + z * split_ystride.
  if constexpr (!M1) {
    if (gridDim.y > 1) {
      const int64_t u0 = (int64_t)blockIdx.y * split_units;
      const int64_t c0 = u0 * (BITS == 4 ? 128 : 64);
      x += c0;
      K = K - c0 < split_units * (BITS == 4 ? 128 : 64) ? K - c0 : split_units * (BITS == 4 ? 128 : 64);
      wq += u0 * 64;
      if constexpr (BITS == 4) sc += u0;
      nunits = nunits - u0 < split_units ? nunits - u0 : split_units;
      y += (int64_t)blockIdx.y * split_ystride;
    }
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int qd = lane >> 4, c = lane & 15;
  const int nT = (int)(nunits * TPU);

  const int64_t ncol0 = (int64_t)blockIdx.x * 16 * NT;
  const uint8_t* wrow[NT];
  const uint16_t* srow[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int64_t n = ncol0 + 16 * t + c;
    const int64_t nl = n < N ? n : N - 1;
    wrow[t] = wq + nl * row_bytes + qd * 16;
    srow[t] = sc + nl * ng;
  }
  const int64_t ub = (int64_t)wave * per_wave;
  const int64_t ue = ub + per_wave < nunits ? ub + per_wave : nunits;

  // Vector-memory counters retire in issue order, so the activation loads of
  // the staging are issued first: waiting for them does not wait for the
  // weights.  Then the first chunk of packed weights (and, for INT4, its group
  // scales) goes in flight, then the staging converts while HBM answers.
  // Each wave stages only the k-steps of its own units, [ub, ue) * TPU, so a
  // wave-level sync replaces a workgroup barrier.  Lane l stages activation
  // row my_m = l / lpr (lpr = 64 / M rounded up to a power of two lanes per
  // row) and its entries e = l % lpr + lpr j < E (k-step tb + e / 4, quad
  // e % 4), so the lanes of a row are one aligned group and the row's scale
  // (its largest |x| over this wave's K-slice) is a reduction within the
  // group.  Slots j < pre_n <= PRE are loaded before the weights; entries past
  // them (or unaligned / K-tail x) are loaded after the weights, where their
  // conversion waits for the weights.  One row: PRE covers one batch of KS
  // units, loaded unconditionally.
  constexpr int PRE1 = KS * TPU / 16 < 1 ? 1 : (KS * TPU / 16 > 4 ? 4 : KS * TPU / 16);
  constexpr int PRE = M1 ? PRE1 : 4;
  const int tb = (int)(ub * TPU), te = (int)(ue * TPU);
  const int E = (te - tb) * 4;
  const int lpr = M1 ? 64 : skinny_lanes_per_row(M);
  const int my_m = M1 ? 0 : lane / lpr;
  const int sub = M1 ? lane : lane & (lpr - 1);
  const bool row_lane = my_m < M;
  const int per_lane = (E + lpr - 1) / lpr;
  const int pre_n = M1 ? PRE : (per_lane < PRE ? per_lane : PRE);
  floatx4 xa4[PRE], xb4[PRE];
  unsigned pre_mask = 0;  // bit j: slot j was pre-loaded
  if constexpr (A_LDS) {
#pragma unroll
    for (int j = 0; j < PRE; j++) {
      if (M1 || j < pre_n) {
        const int e = sub + lpr * j;
        const int T = tb + (e >> 2), q4 = e & 3;
        const bool ok = row_lane && xvec && e < E && kstep_col0<BITS>(T, q4) + 8 <= K;
        pre_mask |= (unsigned)ok << j;
        // A skipped slot reads 32 bytes of the payload instead (rows are at
        // least 64 bytes; x may hold fewer than 8 values).
        const float* src = ok ? x + my_m * ldx + kstep_col0<BITS>(T, q4) : reinterpret_cast<const float*>(wq);
        xa4[j] = reinterpret_cast<const floatx4*>(src)[0];
        xb4[j] = reinterpret_cast<const floatx4*>(src)[1];
      }
    }
  }
  // Keep these loads ahead of the weight loads (an IR-level ordering fence;
  // it emits no instruction and no wait).
  __asm__ volatile("" ::: "memory");

  u32x4 raw[KS][NT];
  uint16_t sv[NT][KS];  // raw fp16 bits: converting at load time would force an early wait
  // INT4 group scales go first: results return in issue order, so a scale
  // issued after the weights would make the first unit's scaling wait for
  // every weight load of the batch.
  if constexpr (BITS == 4) {
#pragma unroll
    for (int t = 0; t < NT; t++) load_scales<KS, SVEC>(srow[t], ub, ue, sv[t]);
  }
  // Unconditional (a branch here would make every later wait conservative):
  // units past ue reload unit ue - 1, which is in [0, nunits) for every wave.
#pragma unroll
  for (int u = 0; u < KS; u++) {
    const int64_t unit = ub + u < ue ? ub + u : ue - 1;
#pragma unroll
    for (int t = 0; t < NT; t++) raw[u][t] = *reinterpret_cast<const u32x4*>(wrow[t] + unit * 64);
  }
  // Nothing that waits for the activation pre-loads may be placed above the
  // weight loads (a conversion there delays every weight load of the wave by
  // one activation-load latency): the pre-loaded registers pass through an
  // empty asm statement here, after the weight loads, so their wait and
  // conversion come after it.
  __asm__ volatile("" ::: "memory");
  if constexpr (A_LDS) {
#pragma unroll
    for (int j = 0; j < PRE; j++) {
      if (M1 || j < pre_n) __asm__ volatile("" : "+v"(xa4[j]), "+v"(xb4[j]));
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  const half8_t* a = xa;
  int ex = 0;  // this lane's row scale exponent (A_LDS staging)
  if constexpr (A_LDS) {
    half8_t* la = reinterpret_cast<half8_t*>(smem);
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < PRE; j++) {
      if ((M1 || j < pre_n) && ((pre_mask >> j) & 1)) {
        const float raw8[8] = {xa4[j][0], xa4[j][1], xa4[j][2], xa4[j][3],
                               xb4[j][0], xb4[j][1], xb4[j][2], xb4[j][3]};
        amax = absmax8(raw8, amax);
      }
    }
    // The row's largest |x| over this wave's slice: the lpr lanes of a row
    // are an aligned group of lanes.
    auto row_exponent = [&](float v) {
      if constexpr (M1) {
        // one row: the exponent is wave-uniform (kept in a scalar register)
        return __builtin_amdgcn_readfirstlane(act_exponent(wave_max_uniform(v)));
      } else {
        return act_exponent(lpr == 64 ? wave_max_uniform(v) : group_max(v, lpr));
      }
    };
    if constexpr (!REM) {
      // The pre-loads cover every entry: convert them from registers.  A slot
      // without a valid pre-load writes its (unused) values to the pad
      // column T = nT of row 0, which no lane reads.
      ex = row_exponent(amax);
      const bool guard = wave_has_inf(amax);
#pragma unroll
      for (int j = 0; j < PRE; j++) {
        if (M1 || j < pre_n) {
          const int e = sub + lpr * j;
          const bool ok = (pre_mask >> j) & 1;
          const float raw8[8] = {xa4[j][0], xa4[j][1], xa4[j][2], xa4[j][3],
                                 xb4[j][0], xb4[j][1], xb4[j][2], xb4[j][3]};
          half8_t hi, lo;
          stage_convert<BITS>(raw8, ex, hi, lo, guard);
          skinny_store<HL>(la, M, pitch, ok ? tb + (e >> 2) : nT, e & 3, ok ? my_m : 0, hi, lo);
        }
      }
    } else {
      // Entries beyond the pre-loads (loaded after the weights, four per lane
      // at a time so their latencies overlap; K-tail entries, which the
      // pre-loads skip, come here with zeros past K) are converted as they
      // arrive, with a provisional exponent of the row-slice: 6 below the
      // exponent of the largest |x| among the pre-loads (among the first four
      // loaded entries when the pre-loads hold no nonzero value: those were
      // converted to exact zeros / NaN, whatever the exponent), so every later
      // entry up to 2^6 times larger still converts without overflow.  Once
      // all are in, the row's true exponent e_true decides: with e_true - ex
      // in [0, 12] the halves are exact to 2^-22 |x| + 2^(-39 + 12) max|x|
      // (fp32-class) and stay; otherwise (a later entry more than ~64x the
      // estimate, or an all-zero estimate) the lanes of that row load and
      // convert their entries again with e_true.
      auto row_max = [&](float v) { return lpr == 64 ? wave_max_uniform(v) : group_max(v, lpr); };
      float raw8[4][8];
      bool need[4];
      int ee[4];
      auto load4 = [&](int j0) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int j = j0 + r;
          ee[r] = sub + lpr * j;
          need[r] = row_lane && j < per_lane && ee[r] < E && !(j < pre_n && ((pre_mask >> j) & 1));
          // row M: stage_load returns zeros without reading
          stage_load<BITS>(x, ldx, M, K, tb + (ee[r] >> 2), ee[r] & 3, need[r] ? my_m : M, xvec, raw8[r]);
        }
      };
      auto store4 = [&](int e_) {
        const bool guard = wave_has_inf(amax);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          if (need[r]) {
            half8_t hi, lo;
            stage_convert<BITS>(raw8[r], e_, hi, lo, guard);
            skinny_store<HL>(la, M, pitch, tb + (ee[r] >> 2), ee[r] & 3, my_m, hi, lo);
          }
        }
      };
      const float pmax = row_max(amax);
      int ex_p = act_exponent(pmax) - 6;
      const bool pguard = wave_has_inf(amax);
#pragma unroll
      for (int j = 0; j < PRE; j++) {
        if (j < pre_n && ((pre_mask >> j) & 1)) {
          const int e = sub + lpr * j;
          const float p8[8] = {xa4[j][0], xa4[j][1], xa4[j][2], xa4[j][3],
                               xb4[j][0], xb4[j][1], xb4[j][2], xb4[j][3]};
          half8_t hi, lo;
          stage_convert<BITS>(p8, ex_p, hi, lo, pguard);
          skinny_store<HL>(la, M, pitch, tb + (e >> 2), e & 3, my_m, hi, lo);
        }
      }
      load4(0);
#pragma unroll
      for (int r = 0; r < 4; r++)
        if (need[r]) amax = absmax8(raw8[r], amax);
      if (!(pmax > 0.0f)) ex_p = act_exponent(row_max(amax)) - 6;
      store4(ex_p);
      for (int j0 = 4; j0 < per_lane; j0 += 4) {
        load4(j0);
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (need[r]) amax = absmax8(raw8[r], amax);
        store4(ex_p);
      }
      const float gmax = row_max(amax);
      const int e_true = act_exponent(gmax);
      const bool keep = !(gmax > 0.0f) || (e_true - ex_p >= 0 && e_true - ex_p <= 12);
      ex = keep ? ex_p : e_true;
      if (!keep) {
        const bool guard = wave_has_inf(amax);
        for (int j = 0; j < per_lane; j++) {
          const int e = sub + lpr * j;
          if (row_lane && e < E) {
            float r8[8];
            stage_load<BITS>(x, ldx, M, K, tb + (e >> 2), e & 3, my_m, xvec, r8);
            half8_t hi, lo;
            stage_convert<BITS>(r8, ex, hi, lo, guard);
            skinny_store<HL>(la, M, pitch, tb + (e >> 2), e & 3, my_m, hi, lo);
          }
        }
      }
    }
    // Only this wave reads what it staged: order its LDS writes before its
    // reads without a workgroup barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    a = la;
  }

  // This lane's activation operand: A-row c of the MFMA.
  bool a_lane;
  const half8_t* a_hi_lane;
  const half8_t* a_lo_lane;
  if constexpr (HL) {
    const int r = c < M ? c : (c >= 8 && c < 8 + M) ? M + c - 8 : -1;
    a_lane = r >= 0;
    a_hi_lane = a + (int64_t)(qd * 2 * M + (a_lane ? r : 0)) * pitch;
    a_lo_lane = a_hi_lane;
  } else {
    a_lane = c < M;
    a_hi_lane = a + (int64_t)(qd * M + (a_lane ? c : 0)) * pitch;
    a_lo_lane = a_hi_lane + (int64_t)4 * M * pitch;
  }

  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  half8_t ah[TPU], al[TPU];
#pragma unroll
  for (int i = 0; i < TPU; i++) { ah[i] = half8_t{}; al[i] = half8_t{}; }

  [[maybe_unused]] const Int4Consts k4 = int4_consts_pinned();
  for (int64_t u0 = ub; u0 < ue; u0 += KS) {
    if (u0 != ub) {
      if constexpr (BITS == 4) {
#pragma unroll
        for (int t = 0; t < NT; t++) load_scales<KS, SVEC>(srow[t], u0, ue, sv[t]);
      }
#pragma unroll
      for (int u = 0; u < KS; u++) {
        const int64_t unit = u0 + u < ue ? u0 + u : ue - 1;
#pragma unroll
        for (int t = 0; t < NT; t++) raw[u][t] = *reinterpret_cast<const u32x4*>(wrow[t] + unit * 64);
      }
    }
#pragma unroll
    for (int u = 0; u < KS; u++) {
      if (u0 + u < ue) {
        const int64_t unit = u0 + u;
        if (a_lane) {
#pragma unroll
          for (int i = 0; i < TPU; i++) {
            ah[i] = a_hi_lane[unit * TPU + i];
            if constexpr (!HL) al[i] = a_lo_lane[unit * TPU + i];
          }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
          if constexpr (BITS == 4) {
            const float s = f16_bits_to_f32(sv[t][u]);
            floatx4 g = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const half8_t b = int4x8_to_half8(raw[u][t][i], k4);
              g = mfma16x16x32(ah[i], b, g);
              if constexpr (!HL) g = mfma16x16x32(al[i], b, g);
            }
            // One row: only accumulator row 0 (x's hi in lane quad 0, its lo
            // in quad 2) is nonzero.
#pragma unroll
            for (int i = 0; i < (M1 ? 1 : 4); i++) acc[t][i] = __builtin_fmaf(s, g[i], acc[t][i]);
          } else {
#pragma unroll
            for (int j = 0; j < 2; j++) {
              const half8_t b = int8x8_to_half8(raw[u][t][2 * j], raw[u][t][2 * j + 1]);
              acc[t] = mfma16x16x32(ah[j], b, acc[t]);
              if constexpr (!HL) acc[t] = mfma16x16x32(al[j], b, acc[t]);
            }
          }
        }
      }
      // Keep each unit's operand loads and conversions next to its MFMAs;
      // hoisting every unit's operands above the first one exhausts VGPRs.
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Cross-wave reduction in a fixed order.  Lane (qd, c) holds output-tile
  // rows 4qd+i, column c of each tile (HL: row m is the hi part of x[m], row
  // m + 8 its lo part), scaled by 2^e_w[m], the wave's exponent of row m
  // (staged in LDS: held by the lanes of row m; staged by the pre-pass: one
  // exponent per row, xexp).  Each wave scales its sums back before the
  // cross-wave sum.  That is exact unless a wave's partial sum lies in the
  // fp32 subnormal range (an output below 2^-126), where each wave's (and
  // each K slice's) partial is rounded once, 2^-150 at most.
  int erow[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 4 * qd + i;
    int mr = HL ? (r < 8 ? r : r - 8) : r;
    mr = mr < M ? mr : M - 1;
    if constexpr (A_LDS) erow[i] = (M1 || lpr == 64) ? ex : __shfl(ex, mr * lpr, 64);
    else erow[i] = xexp[mr];
  }
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int i = 0; i < 4; i++)
      red[((wave * NT + t) * 16 + 4 * qd + i) * 16 + c] = unscale(acc[t][i], erow[i]);
  __syncthreads();
  // Gate / up pairs (NT == 2, weights interleaved by 16-row tiles): tile 0
  // holds gate rows, tile 1 the up rows of the same 16 output columns;
  // y[m][16 b + c] = silu(g) * up.
  if constexpr (NT == 2) {
    if (pairs) {
      for (int o = tid; o < M * 16; o += blockDim.x) {
        const int m = o >> 4, cc = o & 15;
        const int64_t ngate = ncol0 + cc, nup = ngate + 16;
        if (nup < N) {
          float g = 0.0f, u = 0.0f;
          for (int w = 0; w < nwaves; w++) {
            g += red[((w * NT) * 16 + m) * 16 + cc];
            u += red[((w * NT + 1) * 16 + m) * 16 + cc];
            if constexpr (HL) {
              g += red[((w * NT) * 16 + m + 8) * 16 + cc];
              u += red[((w * NT + 1) * 16 + m + 8) * 16 + cc];
            }
          }
          if constexpr (BITS == 8) { g *= f16_bits_to_f32(sc[ngate]); u *= f16_bits_to_f32(sc[nup]); }
          if (bias) { g += bias[ngate]; u += bias[nup]; }
          y[m * ldy + (int64_t)blockIdx.x * 16 + cc] = g / (1.0f + expf(-g)) * u;
        }
      }
      return;
    }
  }
  // y may be null (greedy argmax only).  With argp, the 16 lanes of a row's
  // tile reduce their (logit, column) pairs and lane 0 writes the tile's
  // partial: argp[m * tiles + tile].
  for (int o = tid; o < M * 16 * NT; o += blockDim.x) {
    const int t = o / (M * 16), r = o - t * (M * 16);
    const int m = r >> 4, cc = r & 15;
    const int64_t nn = ncol0 + 16 * t + cc;
    float v = -__builtin_inff();
    int vi = 0x7fffffff;
    if (nn < N) {
      v = 0.0f;
      for (int w = 0; w < nwaves; w++) {
        v += red[((w * NT + t) * 16 + m) * 16 + cc];
        if constexpr (HL) v += red[((w * NT + t) * 16 + m + 8) * 16 + cc];
      }
      if constexpr (BITS == 8) v *= f16_bits_to_f32(sc[nn]);
      if (bias) v += bias[nn];
      if (y) y[m * ldy + nn] = v;
      vi = (int)nn;
    }
    if (argp) {
      arg_reduce16(v, vi);
      if (cc == 0) argp[(int64_t)m * gridDim.x * NT + blockIdx.x * NT + t] = make_int2(__float_as_int(v), vi);
    }
  }
}

// ---------------------------------------------------------------------------
// Workgroup -> (m-tile, n-tile, K split).  Dispatch places block b on XCD
// b % 8, so block b is renumbered r such that each XCD works on one
// contiguous range of r.  r runs through bands of gm m-tiles: within a band
// the m-tile varies fastest, then the n-tile, so one XCD's range touches gm
// m-tiles of activations (sized by the host to stay in that XCD's L2) and
// its weight columns are read by gm workgroups there.  The K split is the
// slowest index.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void gemm_tile(int tiles_m, int tiles_n, int gm, int64_t& tm,
                                          int64_t& tn, int64_t& z) {
  const int64_t nblk = gridDim.x, b = blockIdx.x;
  const int64_t xcd = b % 8, slot = b / 8, q8 = nblk / 8, rem = nblk % 8;
  const int64_t r = xcd < rem ? xcd * (q8 + 1) + slot : rem * (q8 + 1) + (xcd - rem) * q8 + slot;
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  z = r / tiles;
  const int64_t rt = r - z * tiles;
  const int64_t grp = (int64_t)gm * tiles_n;
  const int64_t band = rt / grp, rb = rt - band * grp;
  const int64_t rows = gm < tiles_m - band * gm ? gm : tiles_m - band * gm;
  tm = band * gm + rb % rows;
  tn = rb / rows;
}

// ---------------------------------------------------------------------------
// GEMM path: M > 16 (batched decode, prefill chunks).
//
// stage_rows_kernel converts x once per call into fp16 hi/lo MFMA operand
// planes in the workspace:  entry (plane p, stage st, row m, e) at
//   ((p * nstages + st) * Mp + m) * 16 + e        (16-byte units)
// where stage st covers K columns [128 st, 128 st + 128), e = T * 4 + qd names
// the 8 columns lane quad qd feeds to k-step T of the stage (already permuted
// into operand-slot order), Mp is M rounded up to the row tile, and rows past
// M / columns past K are zeros.  Row m is scaled by 2^rexp[m]; the epilogues
// scale the sums back.
//
// gemm_kernel: workgroup = WN waves side by side along N; wave tile 16*MTW
// rows x 16*NTW columns, so the workgroup tile is BM = 16*MTW by
// BN = 16*NTW*WN.  Per stage the workgroup copies the BM x 128 operand block
// (both planes) into LDS (double-buffered, one barrier per stage) and every
// wave streams its own weight columns from HBM into registers.  The next
// stage's operands, weights and scales are loaded before the current stage's
// MFMAs so their latency hides behind the math.
//
// LDS layout per buffer and plane: row mm holds entry e of activation row
// m0 + mm at mm*16 + (e ^ (mm & 15)).  The XOR makes the 16 rows an MFMA
// operand read touches fall in distinct banks; a thread copies staged entry
// q of the block to LDS entry q (consecutive lanes, consecutive addresses).
//
// Split-K: blockIdx decomposes into (m-tile, n-tile, z); split z covers
// stages [z*spz, (z+1)*spz).  With one split the epilogue writes y; with more
// it writes fp32 partials and splitk_reduce_kernel adds them in z order
// (deterministic).
// ---------------------------------------------------------------------------
template <int BITS, int MTW, int NTW, int WN>
__global__ __launch_bounds__(64 * WN) void gemm_kernel(
    const half8_t* __restrict__ planes, int64_t Mp, int64_t M,
    const uint8_t* __restrict__ wq, const uint16_t* __restrict__ sc, int64_t row_bytes,
    int64_t ng, int64_t nstages, int64_t spz, int tiles_m, int tiles_n, int gm,
    const int* __restrict__ rexp, const float* __restrict__ bias, float* __restrict__ y,
    int64_t ldy, int64_t N, float* __restrict__ part) {
  constexpr int BM = 16 * MTW;
  constexpr int NTHR = 64 * WN;
  constexpr int PLANE = BM * 16;           // LDS entries per plane
  constexpr int CPT = 2 * PLANE / NTHR;    // operand entries each thread copies per stage
  constexpr int RAWN = BITS == 4 ? 1 : 2;  // 16-byte weight loads per n-tile per stage
  static_assert(CPT * NTHR == 2 * PLANE, "operand copy must divide evenly");
  __shared__ half8_t lds[2][2 * PLANE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qd = lane >> 4, c = lane & 15;

  // Tile order: consecutive blocks land on different XCDs, so give each XCD a
  // contiguous range of tiles (m fastest: the m-tiles of one n-tile share
  // their weight columns through that XCD's L2).
  int64_t tm, tn, z;
  gemm_tile(tiles_m, tiles_n, gm, tm, tn, z);
  const int64_t m0 = tm * BM;
  const int64_t n0 = (tn * WN + wave) * (16 * NTW);
  // Lane l holds the exponent of row m0 + l (BM <= 64), loaded now so the
  // epilogue reads it with a lane shuffle instead of a memory round trip.
  const int lane_exp = rexp[m0 + (lane < BM ? lane : 0)];
  const int64_t sb = z * spz;
  const int64_t se = sb + spz < nstages ? sb + spz : nstages;

  const uint8_t* wrow[NTW];
  const uint16_t* srow[NTW];
#pragma unroll
  for (int t = 0; t < NTW; t++) {
    const int64_t n = n0 + t * 16 + c;
    const int64_t nl = n < N ? n : N - 1;
    wrow[t] = wq + nl * row_bytes + qd * 16;
    srow[t] = sc + nl * ng;
  }

  // Operand entry j of this thread: q = tid + j*NTHR -> plane q / PLANE, row
  // mm, physical slot ph; it holds logical entry ph ^ (mm & 15).
  int64_t aoff[CPT];
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int q = tid + j * NTHR;
    const int p = q / PLANE, rr = q % PLANE;
    const int mm = rr >> 4, ph = rr & 15;
    aoff[j] = ((int64_t)p * nstages * Mp + m0 + mm) * 16 + (ph ^ (mm & 15));
  }
  u32x4 areg[CPT];
  auto load_a = [&](int64_t st) {
#pragma unroll
    for (int j = 0; j < CPT; j++)
      areg[j] = reinterpret_cast<const u32x4*>(planes)[aoff[j] + st * Mp * 16];
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int j = 0; j < CPT; j++)
      reinterpret_cast<u32x4*>(lds[buf])[tid + j * NTHR] = areg[j];
  };
  auto load_w = [&](int64_t st, u32x4 (&dst)[NTW][RAWN], uint16_t (&sdst)[NTW]) {
#pragma unroll
    for (int t = 0; t < NTW; t++) {
#pragma unroll
      for (int rr = 0; rr < RAWN; rr++)
        dst[t][rr] = *reinterpret_cast<const u32x4*>(wrow[t] + (st * RAWN + rr) * 64);
      if constexpr (BITS == 4) sdst[t] = srow[t][st];
    }
  };

  floatx4 acc[MTW][NTW];
  floatx4 gacc[MTW][NTW];
#pragma unroll
  for (int i = 0; i < MTW; i++)
#pragma unroll
    for (int t = 0; t < NTW; t++) {
      acc[i][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      gacc[i][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }

  // One stage: prefetch stage sn's operands and weights, run the MFMAs of
  // stage st from LDS buffer buf and registers wc / scur, then copy the
  // prefetched operands into the other buffer.  Called twice per loop trip
  // with the weight registers swapped (ping-pong, no register copies), with
  // no condition inside the trip (a conditional second stage lets the
  // compiler hoist its loads into the first).
  auto stage = [&](int64_t st, int buf, const u32x4 (&wc)[NTW][RAWN], const uint16_t (&scur)[NTW],
                   u32x4 (&wnx)[NTW][RAWN], uint16_t (&snx)[NTW]) {
    // The last stage reloads itself: unconditional loads keep the memory
    // counter waits exact.
    const int64_t sn = st + 1 < se ? st + 1 : st;
    load_a(sn);
    load_w(sn, wnx, snx);
    // Keep the prefetch loads here, ahead of the MFMAs (IR-level and
    // scheduler fences; neither emits an instruction): left alone, the
    // compiler sinks them to their uses at the end of the stage, which
    // serialises load latency and math.
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    const half8_t* la = lds[buf];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      half8_t bw[NTW];
#pragma unroll
      for (int t = 0; t < NTW; t++) {
        if constexpr (BITS == 4) bw[t] = int4x8_to_half8(wc[t][0][i]);
        else bw[t] = int8x8_to_half8(wc[t][i >> 1][2 * (i & 1)], wc[t][i >> 1][2 * (i & 1) + 1]);
      }
#pragma unroll
      for (int mt = 0; mt < MTW; mt++) {
        const int phys = (mt * 16 + c) * 16 + ((i * 4 + qd) ^ c);
        const half8_t ah = la[phys], al = la[PLANE + phys];
#pragma unroll
        for (int t = 0; t < NTW; t++) gacc[mt][t] = mfma16x16x32(ah, bw[t], gacc[mt][t]);
#pragma unroll
        for (int t = 0; t < NTW; t++) gacc[mt][t] = mfma16x16x32(al, bw[t], gacc[mt][t]);
      }
    }
    if constexpr (BITS == 4) {
#pragma unroll
      for (int t = 0; t < NTW; t++) {
        const float s = f16_bits_to_f32(scur[t]);
#pragma unroll
        for (int mt = 0; mt < MTW; mt++) {
#pragma unroll
          for (int i = 0; i < 4; i++) acc[mt][t][i] = __builtin_fmaf(s, gacc[mt][t][i], acc[mt][t][i]);
          gacc[mt][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
    }
    // Copy the prefetched operands only now: the copy waits for their loads,
    // and that wait must not land among the MFMAs.
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    store_a(buf ^ 1);
    __syncthreads();
  };

  u32x4 wa[NTW][RAWN], wb[NTW][RAWN];
  uint16_t sa[NTW], sbv[NTW];
  load_a(sb);
  load_w(sb, wa, sa);
  store_a(0);
  __syncthreads();
  int64_t st = sb;
  for (; st + 1 < se; st += 2) {
    stage(st, 0, wa, sa, wb, sbv);
    stage(st + 1, 1, wb, sbv, wa, sa);
  }
  if (st < se) stage(st, 0, wa, sa, wb, sbv);  // odd stage count

  // Lane (qd, c) holds rows 16*mt + 4*qd + i, column 16*t + c of its wave
  // tile; each row is scaled back by its activation exponent (rows past M
  // are padding: exponent 0 in the planes' padded rows).
  int er[MTW][4];
#pragma unroll
  for (int mt = 0; mt < MTW; mt++)
#pragma unroll
    for (int i = 0; i < 4; i++) er[mt][i] = __shfl(lane_exp, mt * 16 + 4 * qd + i, 64);
#pragma unroll
  for (int t = 0; t < NTW; t++) {
    const int64_t n = n0 + t * 16 + c;
    if (n >= N) continue;
    float s8 = 1.0f, bn = 0.0f;
    if (part == nullptr) {
      if constexpr (BITS == 8) s8 = f16_bits_to_f32(sc[n]);
      if (bias) bn = bias[n];
    }
#pragma unroll
    for (int mt = 0; mt < MTW; mt++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + mt * 16 + 4 * qd + i;
        if (m < M) {
          const float v = BITS == 4 ? acc[mt][t][i] : gacc[mt][t][i];
          if (part == nullptr) y[m * ldy + n] = __builtin_fmaf(unscale(v, er[mt][i]), s8, bn);
          else part[(z * M + m) * N + n] = v;      // still scaled by 2^rexp[m]
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Warp-specialized GEMM (prefill chunks): one producer wave moves each
// stage's operand block (both planes) and the packed weight columns straight
// from memory into an LDS ring of D stages with global_load_lds_dwordx4
// (no registers, no conversion), D - 1 stages ahead of the math; NC
// consumer waves (64 x 64 tiles: BM = 64, BN = 64 NC) only read LDS and run
// MFMAs.  Synchronisation per stage: the producer waits (explicit vmcnt) for
// the stage the consumers are about to read, then one s_barrier; the
// producer's next DMA targets the slot the consumers finished a stage ago.
// The barrier is a bare s_barrier on purpose: a fenced one would make the
// producer wait for every DMA in flight, collapsing the ring to one stage.
//
// LDS per slot: operand planes (hi, lo) in the layout of gemm_kernel, then
// the weights: consumer wave w, n-tile t, window r is one 1 KB block whose
// 16-byte lane slot l holds what MFMA lane l needs (row n0 + 16 t + (l & 15),
// bytes (l >> 4) * 16 of the stage's window r).
// ---------------------------------------------------------------------------
// Shapes (consumer waves of 64 columns, LDS ring depth): 4 consumers with a
// 3-deep ring, or for INT4 grids that fill the GPU without a K split, 7
// consumers (two math waves on most SIMDs, BN = 448) with a 2-deep ring
// (measured 13 % faster there, slower elsewhere: partial 448-column tiles,
// K splits).  INT8 windows need twice the weight ring: 4 consumers with split
// producers (below), weights 3 deep, operands 2 deep -- measured 17-24 %
// faster than one producer with a 2-deep ring at M = 96-512 on the Llama-3-8B
// MLP shapes; for INT4 the deeper weight ring gains nothing (its consumers,
// not the DMA, set the pace).
constexpr int kWsNC = 4, kWsWideNC = 7;
constexpr int64_t kWsWideMinTiles = 256;

__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}

// s_waitcnt with only the vector-memory counter limited to n (n < 64).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// DW > 0: two producer waves, each with its own memory counter -- one moves
// the operand blocks through a 2-deep ring, the other the weights through a
// DW-deep ring, DW - 1 stages ahead.  With one producer both streams share a
// counter that retires in issue order, so waiting for the next operand block
// also waits for every weight DMA issued before it, which caps the weights'
// lead at about two stages whatever the ring depth.
template <int BITS, int D, int NC, int DW = 0>
__global__ __launch_bounds__(64 * (NC + (DW > 0 ? 2 : 1))) void gemm_ws_kernel(
    const half8_t* __restrict__ planes, int64_t Mp, int64_t M,
    const uint8_t* __restrict__ wq, const uint16_t* __restrict__ sc, int64_t row_bytes,
    int64_t ng, int64_t nstages, int64_t spz, int tiles_m, int tiles_n, int gm,
    const int* __restrict__ rexp, const float* __restrict__ bias, float* __restrict__ y,
    int64_t ldy, int64_t N, float* __restrict__ part) {
  constexpr int MTW = 4, NTW = 4, BM = 64;
  constexpr int PLANE = BM * 16;                        // entries per plane
  constexpr int RAWN = BITS == 4 ? 1 : 2;               // 64-byte windows per stage
  constexpr int ABLK = 2 * PLANE / 64;                  // 1 KB operand blocks per stage
  constexpr int WBLK = NC * NTW * RAWN;                 // 1 KB weight blocks per stage
  constexpr int NDMA = ABLK + WBLK;                     // producer DMAs per stage
  constexpr bool SPLIT = DW > 0;
  constexpr int DA = SPLIT ? 2 : D;                     // operand ring depth
  constexpr int DWR = SPLIT ? DW : D;                   // weight ring depth
  static_assert(SPLIT || NDMA * (D - 2) < 64, "vmcnt range");
  static_assert(!SPLIT || WBLK * (DW - 2) < 64, "vmcnt range");
  static_assert((DA * ABLK + DWR * WBLK) * 64 * 16 <= 160 * 1024, "LDS rings exceed 160 KiB");
  __shared__ u32x4 aring[DA * ABLK * 64];
  __shared__ u32x4 wring[DWR * WBLK * 64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool producer = wave >= NC;
  const int qd = lane >> 4, c = lane & 15;

  int64_t tm, tn, z;
  gemm_tile(tiles_m, tiles_n, gm, tm, tn, z);
  const int64_t m0 = tm * BM;
  const int64_t nb = tn * NC * 16 * NTW;                // first column of the workgroup
  // Lane l holds the exponent of row m0 + l (BM = 64), loaded now so the
  // epilogue reads it with a lane shuffle instead of a memory round trip.
  const int lane_exp = rexp[m0 + lane];
  const int64_t sb = z * spz;
  const int64_t se = sb + spz < nstages ? sb + spz : nstages;
  const int64_t nst = se - sb;

  // Producer addressing: operand block j -> plane j / (BM/4), rows 4 (j % (BM/4)) + (lane >> 4);
  // weight block (w, t, rr) -> row nb + 64 w + 16 t + (lane & 15), byte (lane >> 4) * 16.
  auto issue_a = [&](int64_t st, int sl) {
    u32x4* base = aring + sl * ABLK * 64;
#pragma unroll
    for (int j = 0; j < ABLK; j++) {
      const int p = j / (BM / 4), mm = (j % (BM / 4)) * 4 + (lane >> 4), ph = lane & 15;
      const int64_t e = ((p * nstages + st) * Mp + m0 + mm) * 16 + (ph ^ (mm & 15));
      dma16(planes + e, base + j * 64);
    }
  };
  auto issue_w = [&](int64_t st, int sl) {
    u32x4* base = wring + sl * WBLK * 64;
#pragma unroll
    for (int w = 0; w < NC; w++)
#pragma unroll
      for (int t = 0; t < NTW; t++) {
        const int64_t n = nb + 64 * w + 16 * t + (lane & 15);
        const uint8_t* src = wq + (n < N ? n : N - 1) * row_bytes + (lane >> 4) * 16;
#pragma unroll
        for (int rr = 0; rr < RAWN; rr++)
          dma16(src + (st * RAWN + rr) * 64, base + ((w * NTW + t) * RAWN + rr) * 64);
      }
  };

  floatx4 acc[MTW][NTW];
#pragma unroll
  for (int i = 0; i < MTW; i++)
#pragma unroll
    for (int t = 0; t < NTW; t++) acc[i][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t n0 = nb + 64 * (producer ? 0 : wave);
  const uint16_t* srow[NTW];
#pragma unroll
  for (int t = 0; t < NTW; t++) {
    const int64_t n = n0 + 16 * t + c;
    srow[t] = sc + (n < N ? n : N - 1) * ng;
  }

  // Producer and consumers run separate loops with the same number of
  // barriers (one per stage), so neither path's registers burden the other.
  if (producer) {
    if constexpr (SPLIT) {
      if (wave == NC) {                           // operand blocks, one stage ahead
        issue_a(sb, 0);
        for (int64_t s = 0; s < nst; s++) {
          wait_vmcnt<0>();                        // stage s has landed
          __builtin_amdgcn_s_barrier();
          const int64_t k = s + 1;                // into the slot read a stage ago
          issue_a(sb + (k < nst ? k : nst - 1), (int)(k & 1));
        }
      } else {                                    // weights, DW - 1 stages ahead
#pragma unroll
        for (int k = 0; k < DW - 1; k++) issue_w(sb + (k < nst ? k : nst - 1), k);
        for (int64_t s = 0; s < nst; s++) {
          wait_vmcnt<WBLK * (DW - 2)>();          // stage s has landed
          __builtin_amdgcn_s_barrier();
          const int64_t k = s + DW - 1;
          issue_w(sb + (k < nst ? k : nst - 1), (int)(k % DW));
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < D - 1; k++) {
        issue_a(sb + (k < nst ? k : nst - 1), k);
        issue_w(sb + (k < nst ? k : nst - 1), k);
      }
      for (int64_t s = 0; s < nst; s++) {
        wait_vmcnt<NDMA * (D - 2)>();             // stage s has landed
        __builtin_amdgcn_s_barrier();
        const int64_t k = s + D - 1;              // into the slot read a stage ago
        issue_a(sb + (k < nst ? k : nst - 1), (int)(k % D));
        issue_w(sb + (k < nst ? k : nst - 1), (int)(k % D));
      }
    }
    return;
  }

  uint16_t scur[NTW];
  if constexpr (BITS == 4) {
#pragma unroll
    for (int t = 0; t < NTW; t++) scur[t] = srow[t][sb];
  }
  for (int64_t s = 0; s < nst; s++) {
    wait_lgkmcnt0();                              // this wave's reads of stage s - 1 are done
    __builtin_amdgcn_s_barrier();
    uint16_t snx[NTW];
    if constexpr (BITS == 4) {
      const int64_t sn = sb + (s + 1 < nst ? s + 1 : s);
#pragma unroll
      for (int t = 0; t < NTW; t++) snx[t] = srow[t][sn];
    }
    const u32x4* wbase = wring + (int)(s % DWR) * WBLK * 64;
    const half8_t* la = reinterpret_cast<const half8_t*>(aring + (int)(s % DA) * ABLK * 64);
    u32x4 wr[NTW][RAWN];
#pragma unroll
    for (int t = 0; t < NTW; t++)
#pragma unroll
      for (int rr = 0; rr < RAWN; rr++)
        wr[t][rr] = wbase[((wave * NTW + t) * RAWN + rr) * 64 + lane];
    float sf[NTW];
    if constexpr (BITS == 4) {
#pragma unroll
      for (int t = 0; t < NTW; t++) { sf[t] = f16_bits_to_f32(scur[t]); scur[t] = snx[t]; }
    }
    // k-step outer, m-tile inner: only one k-step's B operands are converted
    // ahead of its MFMAs, so converting the next k-step (and reading its A
    // fragments) overlaps the current k-step's 8 MTW MFMAs instead of all
    // conversion running before the stage's first MFMA.  INT4 sums each
    // group (this stage) apart in g and applies the group scale at the end.
    floatx4 g[MTW][NTW];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      half8_t bw[NTW];
#pragma unroll
      for (int t = 0; t < NTW; t++) {
        if constexpr (BITS == 4) bw[t] = int4x8_to_half8(wr[t][0][i]);
        else bw[t] = int8x8_to_half8(wr[t][i >> 1][2 * (i & 1)], wr[t][i >> 1][2 * (i & 1) + 1]);
      }
#pragma unroll
      for (int mt = 0; mt < MTW; mt++) {
        const int phys = (mt * 16 + c) * 16 + ((i * 4 + qd) ^ c);
        const half8_t ah = la[phys], al = la[PLANE + phys];
#pragma unroll
        for (int t = 0; t < NTW; t++) {
          const floatx4 g0 = i > 0 ? g[mt][t] : (BITS == 4 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : acc[mt][t]);
          g[mt][t] = mfma16x16x32(ah, bw[t], g0);
        }
#pragma unroll
        for (int t = 0; t < NTW; t++) g[mt][t] = mfma16x16x32(al, bw[t], g[mt][t]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MTW; mt++)
#pragma unroll
      for (int t = 0; t < NTW; t++) {
        if constexpr (BITS == 4) {
#pragma unroll
          for (int i = 0; i < 4; i++) acc[mt][t][i] = __builtin_fmaf(sf[t], g[mt][t][i], acc[mt][t][i]);
        } else {
          acc[mt][t] = g[mt][t];
        }
      }
  }

  int er[MTW][4];
#pragma unroll
  for (int mt = 0; mt < MTW; mt++)
#pragma unroll
    for (int i = 0; i < 4; i++) er[mt][i] = __shfl(lane_exp, mt * 16 + 4 * qd + i, 64);
#pragma unroll
  for (int t = 0; t < NTW; t++) {
    const int64_t n = n0 + t * 16 + c;
    if (n >= N) continue;
    float s8 = 1.0f, bn = 0.0f;
    if (part == nullptr) {
      if constexpr (BITS == 8) s8 = f16_bits_to_f32(sc[n]);
      if (bias) bn = bias[n];
    }
#pragma unroll
    for (int mt = 0; mt < MTW; mt++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + mt * 16 + 4 * qd + i;
        if (m < M) {
          const float v = acc[mt][t][i];
          if (part == nullptr) y[m * ldy + n] = __builtin_fmaf(unscale(v, er[mt][i]), s8, bn);
          else part[(z * M + m) * N + n] = v;      // still scaled by 2^rexp[m]
        }
      }
    }
  }
}

// Row argmax, pass 1 over materialised logits: block (chunk, m) reduces
// columns [chunk * 4096, +4096) of row m to argp[m * chunks + chunk].
constexpr int kArgChunk = 4096;
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ y, int64_t ldy,
                                                             int64_t N, int2* __restrict__ argp) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int64_t m = blockIdx.y, c0 = (int64_t)blockIdx.x * kArgChunk;
  float v = -__builtin_inff();
  int vi = 0x7fffffff;
  // All 16 loads of a thread are issued before any is compared (unrolled,
  // column clamped into the row), so their latencies overlap.
  float a[kArgChunk / 256];
#pragma unroll
  for (int j = 0; j < kArgChunk / 256; j++) {
    const int64_t col = c0 + threadIdx.x + 256 * j;
    a[j] = y[m * ldy + (col < N ? col : N - 1)];
  }
#pragma unroll
  for (int j = 0; j < kArgChunk / 256; j++) {
    const int64_t col = c0 + threadIdx.x + 256 * j;
    if (col < N && arg_better(a[j], (int)col, v, vi)) { v = a[j]; vi = (int)col; }
  }
  arg_reduce16(v, vi);
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(vi, off);
    if (arg_better(ov, oi, v, vi)) { v = ov; vi = oi; }
  }
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = vi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++)
      if (arg_better(sv[w], si[w], v, vi)) { v = sv[w]; vi = si[w]; }
    argp[m * gridDim.x + blockIdx.x] = make_int2(__float_as_int(v), vi);
  }
}

// Row argmax, pass 2: block m reduces the row's `parts` partials to tokens[m].
__global__ __launch_bounds__(1024) void argmax_final_kernel(const int2* __restrict__ argp, int64_t parts,
                                                            int64_t* __restrict__ tokens) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int64_t m = blockIdx.x;
  float v = -__builtin_inff();
  int vi = 0x7fffffff;
  // Eight partials per thread per round, all loaded before any is compared.
  for (int64_t j0 = threadIdx.x; j0 < parts; j0 += 8 * 1024) {
    int2 q[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int64_t j = j0 + 1024 * u;
      q[u] = argp[m * parts + (j < parts ? j : parts - 1)];
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const float a = __int_as_float(q[u].x);
      if (j0 + 1024 * u < parts && arg_better(a, q[u].y, v, vi)) { v = a; vi = q[u].y; }
    }
  }
  arg_reduce16(v, vi);
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(vi, off);
    if (arg_better(ov, oi, v, vi)) { v = ov; vi = oi; }
  }
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = vi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; w++)
      if (arg_better(sv[w], si[w], v, vi)) { v = sv[w]; vi = si[w]; }
    tokens[m] = vi;
  }
}

// y[m, n] = (sum over z of part[z, m, n]) (* INT8 row scale) + bias, z in
// order.  Partial z of row m is scaled by 2^pexp[z * pz + m] (pz = 0: one
// exponent per row for every slice; pexp null: unscaled partials); the
// slices meet in the domain of the row's smallest exponent E and the sum is
// scaled back by 2^-E once.
// VEC: four consecutive n per thread (N % 4 == 0, y rows 16-byte aligned).
template <int BITS, bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int S,
                                                            int64_t M, int64_t N,
                                                            const int* __restrict__ pexp, int64_t pz,
                                                            const uint16_t* __restrict__ sc,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ y, int64_t ldy) {
  constexpr int V = VEC ? 4 : 1;
  const int64_t total = M * N;
  for (int64_t o = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V; o < total;
       o += (int64_t)gridDim.x * blockDim.x * V) {
    const int64_t m = o / N, n = o - m * N;
    int e = pexp ? pexp[m] : 0;
    for (int zz = 1; zz < S && pz != 0; zz++) e = min(e, pexp[zz * pz + m]);
    float v[V];
#pragma unroll
    for (int u = 0; u < V; u++) v[u] = 0.0f;
    // Slices are added in order; the loads of up to 8 slices are issued
    // before their adds, so 8 slices cost one memory round trip.
    auto add = [&](const float4& p, int zz) {
      const int d = pz != 0 ? e - pexp[zz * pz + m] : 0;
      v[0] += __builtin_amdgcn_ldexpf(p.x, d);
      if constexpr (VEC) {
        v[1] += __builtin_amdgcn_ldexpf(p.y, d);
        v[2] += __builtin_amdgcn_ldexpf(p.z, d);
        v[3] += __builtin_amdgcn_ldexpf(p.w, d);
      }
    };
    auto load = [&](int zz) {
      if constexpr (VEC) return *reinterpret_cast<const float4*>(part + zz * total + o);
      else return float4{part[zz * total + o], 0.0f, 0.0f, 0.0f};
    };
    int zz = 0;
    for (; zz + 8 <= S; zz += 8) {
      float4 p[8];
#pragma unroll
      for (int j = 0; j < 8; j++) p[j] = load(zz + j);
#pragma unroll
      for (int j = 0; j < 8; j++) add(p[j], zz + j);
    }
    if (zz < S) {
      float4 p[8];
#pragma unroll
      for (int j = 0; j < 8; j++) p[j] = load(zz + j < S ? zz + j : zz);
#pragma unroll
      for (int j = 0; j < 8; j++)
        if (zz + j < S) add(p[j], zz + j);
    }
#pragma unroll
    for (int u = 0; u < V; u++) {
      float s8 = 1.0f;
      if constexpr (BITS == 8) s8 = f16_bits_to_f32(sc[n + u]);
      v[u] = __builtin_fmaf(unscale(v[u], e), s8, bias ? bias[n + u] : 0.0f);
    }
    if constexpr (VEC) *reinterpret_cast<float4*>(y + m * ldy + n) = float4{v[0], v[1], v[2], v[3]};
    else y[m * ldy + n] = v[0];
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
constexpr int kSkinnyHLMaxM = 8;             // hi/lo in separate MFMA rows up to M = 8
constexpr int kSkinnyMaxWaves = 16;
constexpr int kSkinnyMaxWaves16 = 8;          // with 16-unit batches (skinny_max_threads)
constexpr int64_t kSkinnyMinWaves = 2048;      // 8 waves per CU across 256 CUs
constexpr int64_t kSkinnyMaxTotalWaves = 12288; // 48 per CU
constexpr int kSkinnyNTMinM = 2;                // several 16-column tiles per workgroup from this M
constexpr int kSkinnyNT4MinM = 5;               // ... four of them only from this M
constexpr int64_t kSkinnyMinGroups = 192;
constexpr int64_t kSkinnyOneRound = 4096;       // waves resident at once (4 per SIMD x 1024 SIMDs)
constexpr int64_t kSkinnyLdsA = 160 * 1024;  // LDS per CU (gfx950), all usable by one workgroup
constexpr int64_t kSkinnyLdsSmall = 64 * 1024;  // staging this small never limits residency
constexpr int64_t kSkinnyLdsTwo = 80 * 1024;    // two workgroups per CU: LDS even over rounds
constexpr int64_t kSkinnySplitMinM = 3;         // K split across workgroups from this M
constexpr int64_t kSkinnySplitMinK = 8192;      // ... and this K
// From this M the K split aims at two workgroups per CU (one below): down_proj
// at M = 5 / 6 went 29.7 / 28.9 -> 20.2 / 20.4 us INT8, 23.9 / 22.2 -> 19.5 /
// 19.8 us INT4 (5 -> 8 slices); at M = 3 / 4 INT4 loses 2 us.
constexpr int64_t kSkinnySplit2MinM = 5;
constexpr int64_t kCUs = 256;
constexpr int kGemmWN = 4;                    // waves per workgroup (one column strip each)
// INT8 on very wide N (the wide-tile case below, i.e. lm_head) runs 8 waves
// of four tiles (BN = 512) with the two-per-CU split target (a 2-way K split
// on [128256 x 4096]): measured 132.8 -> 119.4 us at M = 17, 140.5 -> 133.3
// us at M = 32 (8 waves without the split: slower); INT4 loses there.
constexpr int kGemmWideWN8 = 8;
// 16-column tiles per wave: two (BN = 128) unless that gives more than
// kGemmNarrowMaxTiles column tiles, then four (BN = 256).  Measured at M =
// 17-32 on the Llama-3-8B shapes: BN = 128 takes 2-4 us off down / o /
// q+k+v (twice the workgroups, half the K splits and partials), BN = 256
// is faster for lm_head (1002 narrow tiles).
constexpr int64_t kGemmNarrowMaxTiles = 512;
constexpr int64_t kGemmTargetBlocks = 512;  // two resident workgroups per CU (INT4)
constexpr int64_t kGemmTargetBlocks8 = 256; // INT8: one per CU (fewer K splits; measured
                                            // 1-3 us faster at M = 17-64, INT4 loses)
constexpr int64_t kGemmMinStages = 4;       // stages per K split, at least
constexpr int64_t kGemmWsMinM = 33;         // warp-specialized DMA kernel from this M (INT4)
// INT8 keeps gemm_kernel (64-row tiles above M = 32) up to M = 64: measured
// at M = 33-64 on the Llama-3-8B shapes it is 2-13 us faster there (down,
// gate/up, o, q+k+v, lm_head); for INT4 it loses on down and gate/up.
constexpr int64_t kGemmWsMinM8 = 65;        // the same for INT8
constexpr int64_t kGemmWsTargetBlocks = 256;  // one resident workgroup per CU (LDS ring)

inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

enum class Path { Skinny, Gemm, Generic };

struct Plan;
struct GemmWs {
  size_t rexp_off = 0, part_off = 0, total = 0;
};
GemmWs gemm_ws_layout(const Plan& p);

struct Plan {
  Path path;
  int ks = 0;           // skinny: units per load batch (template)
  int nt = 1;           // skinny: 16-column tiles per workgroup (template)
  int waves = 0;        // skinny: waves per workgroup
  int64_t per_wave = 0; // skinny: units per wave
  bool a_lds = false;   // skinny: activations staged in LDS by the workgroup
  bool hl = false;      // skinny: hi/lo halves in separate MFMA rows
  bool svec = false;    // skinny INT4: vector loads of KS consecutive group scales
  int64_t nunits = 0;   // INT4 groups / INT8 windows per row
  int64_t nT = 0;       // k-steps
  int mtw = 0;          // gemm: 16-row m-tiles per wave (BM = 16 * mtw)
  int ntw = 4;          // gemm: 16-column tiles per wave (BN = 16 * ntw * wn)
  int wn = kGemmWN;     // gemm: waves per workgroup
  int64_t tiles_m = 0;  // gemm: workgroup tiles along M
  int64_t tiles_n = 0;  // gemm: workgroup tiles along N
  int64_t nstages = 0;  // gemm: 128-column K stages
  int64_t spz = 0;      // gemm: stages per K split
  int64_t splits = 1;   // gemm: K splits (partials + ordered reduction when > 1)
  int gm = 1;           // gemm: m-tiles per band of the workgroup order
  int wsnc = 0;         // gemm: consumer waves of the warp-specialized kernel
  bool wsdw = false;    // gemm: warp-specialized kernel with split producers (deep weight ring)
  bool pairs = false;   // skinny: gate / up tile pairs, silu(gate) * up epilogue
  int64_t mpad = 0;     // gemm: operand-plane rows (M rounded up to the row tile)
  bool wspec = false;   // gemm: warp-specialized DMA kernel (prefill chunks)
  int64_t pitch = 0;    // skinny: entries per (quad, A-row) in the lane-major layout
  int64_t ksplit = 1;   // skinny: K slices across workgroup rows (partials + reduction when > 1)
  int64_t split_units = 0;  // skinny: units per K slice
  size_t ws = 0;        // workspace bytes
  int64_t m = 0, n = 0; // the linear's batch rows and out_features
};

// pairs: N rows interleave gate and up weights by 16-row tiles; a skinny
// plan then takes exactly two tiles per wave (one gate / up pair).
// split: the caller can take a K-split skinny plan (plain linear only).
Plan make_plan(int bits, int64_t m, int64_t n, int64_t k, int64_t g, int64_t kp, bool pairs = false,
               bool split = false) {
  Plan p;
  p.m = m;
  p.n = n;
  const bool tiled = bits == 4 ? (g == 128) : (k % 64 == 0);
  if (!tiled) { p.path = Path::Generic; return p; }
  p.nunits = bits == 4 ? kp / 128 : k / 64;
  p.nT = p.nunits * (bits == 4 ? 4 : 2);
  if (m <= kSkinnyMaxM) {
    p.path = Path::Skinny;
    p.hl = m <= kSkinnyHLMaxM;
    // Units per wave: a power of two (so every wave's first unit is aligned for
    // vector scale loads), at most 16 waves per workgroup.  Measured rule:
    // 8-unit (8 KB per wave) batches when that still gives >= 2048 waves
    // (8 per CU); smaller batches for small launches; 16-unit batches only
    // when 8 would need more than 16 waves per workgroup or > 12288 waves.
    // Tiles per workgroup: each workgroup stages all of x for its columns, so
    // wider workgroups cut that traffic (it is M x the weights' own at 16
    // columns); keep at least 192 workgroups for parallelism.
    p.nt = 1;
    if (m >= kSkinnyNTMinM) {
      const int64_t t16 = (n + 15) / 16;
      p.nt = t16 / 4 >= kSkinnyMinGroups ? 4 : (t16 / 2 >= kSkinnyMinGroups ? 2 : 1);
    }
    if (pairs) {
      p.nt = 2;
      p.pairs = true;
    }
    const int64_t tpu = bits == 4 ? 4 : 2;
    // K split (tall K, M >= 3): every workgroup stages all of x for its
    // columns, i.e. M x K activations per 16 * NT columns.  When that cannot
    // stay in LDS with the grid resident, or the shape allows fewer than 4
    // tiles per workgroup, workgroups take 4 tiles and a K slice small enough
    // that its staging stays <= 64 KiB, with enough slices for one workgroup
    // per CU; partial sums are added in slice order by a reduction.  The
    // reduction launch and the partials cost ~3 us, so (measured on the
    // Llama-3-8B shapes) this pays only from K = 8192 and M = 3 (down_proj
    // at M = 3: 23.7 -> 19.7 us INT8; at M = 8: 34 -> 23 us INT8, 28 -> 23 us
    // INT4); shorter K, and M = 2, lose.
    int64_t units = p.nunits;
    if (split && m >= kSkinnySplitMinM && k >= kSkinnySplitMinK && !pairs) {
      const int64_t groups = (n + 16 * p.nt - 1) / (16 * p.nt);
      const int64_t full = 128 * ((p.nT + 1) | 1) * m;
      const bool fits = full <= kSkinnyLdsSmall ||
                        (full <= kSkinnyLdsA && (kSkinnyLdsA / full) * kCUs >= groups);
      if (!fits || p.nt < 4) {
        const int64_t tiles4 = (n + 63) / 64;
        auto slice = [&](int64_t s) { return (p.nunits + s - 1) / s; };
        int64_t s = 1;
        while (s < p.nunits &&
               (tiles4 * s < (m >= kSkinnySplit2MinM ? 2 : 1) * kCUs ||
                128 * ((slice(s) * tpu + 1) | 1) * m > kSkinnyLdsSmall))
          ++s;
        if (s > 1) {
          p.nt = 4;
          units = slice(s);
          p.ksplit = (p.nunits + units - 1) / units;
        }
      }
    }
    p.split_units = units;
    const int64_t ntiles = (n + 16 * p.nt - 1) / (16 * p.nt) * p.ksplit;
    auto waves_for = [&](int64_t pw) { return ntiles * ((units + pw - 1) / pw); };
    int64_t best_pw = 2;
    for (int64_t pw = 8; pw >= 2; pw /= 2) {
      if (waves_for(pw) >= kSkinnyMinWaves) { best_pw = pw; break; }
    }
    if ((units + 7) / 8 > kSkinnyMaxWaves || waves_for(8) > kSkinnyMaxTotalWaves) best_pw = 16;
    while ((units + best_pw - 1) / best_pw > kSkinnyMaxWaves && best_pw < 16) best_pw *= 2;
    p.per_wave = best_pw;
    // Below M = 5, two tiles per workgroup instead of four, in 4-unit
    // batches: the staging four tiles share is small there and twice the
    // workgroups balance better (measured at M = 2 / 4, INT4: gate+up
    // [28672 x 4096] 21.4 -> 17.3 / 22.5 -> 20.6 us, gate [14336 x 4096]
    // 12.3 -> 10.6 us at M = 2).
    if (p.nt == 4 && m >= 2 && m < kSkinnyNT4MinM && !pairs && p.ksplit == 1) {
      p.nt = 2;
      best_pw = std::max<int64_t>(best_pw, 4);
      p.per_wave = best_pw;
    }
    const int64_t maxw = std::min<int64_t>(best_pw, 16 / p.nt) * p.nt >= 16 ? kSkinnyMaxWaves16
                                                                           : kSkinnyMaxWaves;
    p.waves = (int)std::min<int64_t>((units + best_pw - 1) / best_pw, maxw);
    if ((int64_t)p.waves * best_pw < units)          // long K: several KS-unit batches
      p.per_wave = (units + p.waves - 1) / p.waves;
    p.ks = (int)std::min<int64_t>(best_pw, 16 / p.nt);
    // M = 1: two tiles per wave in 4-unit batches and 8 waves per workgroup
    // halve the activation staging per column (it reads all of x per
    // workgroup) without fattening the waves, when that keeps >= 192
    // workgroups and fits one round of resident waves.  Measured on the
    // Llama-3-8B shapes: gate / up and q+k+v gain 0.5-1.6 us per launch;
    // launches needing a second round of waves (gate+up) or leaving CUs idle
    // (o_proj, down_proj) lose.
    if (m == 1) {
      int64_t pw2 = 1;
      while (pw2 * 8 < p.nunits) pw2 *= 2;
      const int64_t wpg = (p.nunits + pw2 - 1) / pw2;
      const int64_t groups = ((n + 15) / 16 + 1) / 2;
      if (pw2 >= 4 && wpg <= 8 && groups >= kSkinnyMinGroups && groups * wpg <= kSkinnyOneRound) {
        p.nt = 2;
        p.per_wave = pw2;
        p.waves = (int)wpg;
        p.ks = 4;
      }
    }
    p.svec = bits == 4 && p.per_wave % p.ks == 0 && (kp / 128) % p.ks == 0 && units % p.ks == 0;
    // An odd pitch puts the four lane quads of an LDS row in different banks;
    // column nT is a pad column (written with unused values, never read).
    p.pitch = (units * tpu + 1) | 1;
    // Staged activations: 2 halves x 16 B x 4 quads per entry.  Above 64 KiB
    // they limit how many workgroups a CU holds; stage in LDS then only if
    // two still fit a CU (<= 80 KiB: M = 4 at K = 4096) or the whole grid is
    // resident at once (else, with one workgroup per CU and a second round
    // waiting, measured slower than staging by a pre-pass).
    {
      const int64_t abytes = 128 * p.pitch * m;
      const int64_t groups = (n + 16 * p.nt - 1) / (16 * p.nt);
      p.a_lds = abytes <= kSkinnyLdsSmall || abytes <= kSkinnyLdsTwo ||
                (abytes <= kSkinnyLdsA && (kSkinnyLdsA / abytes) * kCUs >= groups);
    }
    if (!p.a_lds) p.pitch = p.nT;
    // Pre-pass staging: the staged rows, then one scale exponent per row.
    p.ws = p.a_lds ? 0 : align256((size_t)(128 * p.pitch * m)) + (size_t)(4 * m);
    if (p.ksplit > 1) p.ws = (size_t)(4 * p.ksplit * m * n);   // partials (staging is in LDS)
    return p;
  }
  const int64_t keff = p.nT * 32;
  if (keff % 128 != 0) { p.path = Path::Generic; return p; }
  p.path = Path::Gemm;
  p.wspec = m >= (bits == 8 ? kGemmWsMinM8 : kGemmWsMinM);
  p.mtw = (m <= 32 && !p.wspec) ? 2 : 4;
  p.tiles_m = (m + 16 * p.mtw - 1) / (16 * p.mtw);
  if (p.wspec) {
    const int64_t wide = (n + 64 * kWsWideNC - 1) / (64 * kWsWideNC);
    p.wsnc = bits == 4 && p.tiles_m * wide >= kWsWideMinTiles ? kWsWideNC : kWsNC;
    p.wsdw = bits == 8;
  }
  if (!p.wspec) {
    p.ntw = (n + 16 * 2 * kGemmWN - 1) / (16 * 2 * kGemmWN) <= kGemmNarrowMaxTiles ? 2 : 4;
    if (p.ntw == 4 && bits == 8 && p.mtw == 2) p.wn = kGemmWideWN8;
  }
  const int64_t bn = p.wspec ? 64 * p.wsnc : 16 * p.ntw * p.wn;
  p.tiles_n = (n + bn - 1) / bn;
  p.nstages = keff / 128;
  // Split K only as far as needed to give every CU two workgroups.
  const int64_t tiles = p.tiles_m * p.tiles_n;
  const int64_t target = p.wspec ? kGemmWsTargetBlocks
                                 : (bits == 8 && p.wn != kGemmWideWN8 ? kGemmTargetBlocks8 : kGemmTargetBlocks);
  int64_t s = 1;
  if (tiles < target)
    s = std::max<int64_t>(1, std::min(target / tiles, p.nstages / kGemmMinStages));
  p.spz = (p.nstages + s - 1) / s;
  p.splits = (p.nstages + p.spz - 1) / p.spz;
  p.mpad = p.tiles_m * 16 * p.mtw;
  // Bands of m-tiles whose operand planes (BM rows x K x 4 bytes each) fit
  // about 2 MiB of an XCD's L2.
  {
    const int64_t per_mtile = 16 * p.mtw * keff * 4;
    p.gm = (int)std::max<int64_t>(1, std::min<int64_t>(p.tiles_m, (2 << 20) / per_mtile));
  }
  // Operand planes (2 x 16 bytes per entry), the row exponents, then
  // split-K partials (gemm_ws_layout).
  p.ws = gemm_ws_layout(p).total;
  return p;
}

GemmWs gemm_ws_layout(const Plan& p) {
  GemmWs w;
  w.rexp_off = align256((size_t)(2 * 16 * p.nstages * p.mpad * 16));
  w.part_off = align256(w.rexp_off + (size_t)(4 * p.mpad));
  w.total = p.splits > 1 ? w.part_off + (size_t)(4 * p.splits * p.m * p.n) : w.rexp_off + (size_t)(4 * p.mpad);
  return w;
}

inline bool x_vectorizable(const float* x, int64_t ldx, int64_t k) {
  return (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (ldx % 4 == 0) && k >= 8;
}

template <int BITS, bool LDS, bool HL, bool SVEC, bool M1, bool REM>
void launch_skinny_ks(const Plan& p, dim3 grid, dim3 block, size_t shm, hipStream_t st,
                      const float* x, int64_t ldx, int64_t m, int64_t k, bool xvec,
                      const uint8_t* wq, const uint16_t* sc, int64_t row_bytes, int64_t ng,
                      const half8_t* xa, const int* xexp, const float* bias, float* y,
                      int64_t ldy, int64_t n, int2* argp) {
  const int pairs = p.pairs ? 1 : 0;
#define KQ_SKINNY(KS_, NT_)                                                                   \
  skinny_kernel<BITS, KS_, NT_, LDS, HL, SVEC, M1, REM><<<grid, block, shm, st>>>(            \
      x, ldx, (int)m, k, xvec, wq, sc, row_bytes, ng, p.nunits, p.per_wave, (int)p.pitch, xa, \
      xexp, bias, y, ldy, n, argp, pairs, p.split_units, m * n)
  if (p.nt == 4) {
    if (p.ks == 2) KQ_SKINNY(2, 4); else KQ_SKINNY(4, 4);
  } else if (p.nt == 2) {
    switch (p.ks) {
      case 2: KQ_SKINNY(2, 2); break;
      case 4: KQ_SKINNY(4, 2); break;
      default: KQ_SKINNY(8, 2); break;
    }
  } else {
    switch (p.ks) {
      case 2: KQ_SKINNY(2, 1); break;
      case 4: KQ_SKINNY(4, 1); break;
      case 8: KQ_SKINNY(8, 1); break;
      default: KQ_SKINNY(16, 1); break;
    }
  }
#undef KQ_SKINNY
}

template <int BITS>
int launch_skinny(const Plan& p, const float* x, int64_t ldx, int64_t m, int64_t k,
                  const uint8_t* wq, const uint16_t* sc, int64_t row_bytes, int64_t ng,
                  const float* bias, float* y, int64_t ldy, int64_t n, void* ws, hipStream_t st,
                  int2* argp = nullptr) {
  const bool xvec = x_vectorizable(x, ldx, k);
  const half8_t* xa = nullptr;
  const int* xexp = nullptr;
  if (!p.a_lds) {
    // Staged by a pre-pass, one workgroup per row (row scale over all of K).
    half8_t* a = static_cast<half8_t*>(ws);
    int* e = reinterpret_cast<int*>(static_cast<char*>(ws) + align256((size_t)(128 * p.pitch * m)));
    if (p.hl)
      stage_rows_kernel<BITS, false, true><<<(unsigned)m, 256, 0, st>>>(x, ldx, (int)m, k, (int)p.nT, p.pitch, 0, xvec, a, e);
    else
      stage_rows_kernel<BITS, false, false><<<(unsigned)m, 256, 0, st>>>(x, ldx, (int)m, k, (int)p.nT, p.pitch, 0, xvec, a, e);
    xa = a;
    xexp = e;
  }
  const size_t red = (size_t)p.waves * p.nt * 256 * sizeof(float);
  const size_t abytes = p.a_lds ? (size_t)(128 * p.pitch * m) : 0;
  const size_t shm = std::max(red, abytes);
  const dim3 grid((unsigned)((n + 16 * p.nt - 1) / (16 * p.nt)), (unsigned)p.ksplit);
  // K split: the slices write partials (row scale applied, no bias) to the
  // workspace, [slice][m][n]; the reduction adds them in slice order + bias.
  float* const y_out = y;
  const int64_t ldy_out = ldy;
  const float* const bias_out = bias;
  if (p.ksplit > 1) {
    y = static_cast<float*>(ws);
    ldy = n;
    bias = nullptr;
  }
  const dim3 block((unsigned)(64 * p.waves));
  const bool svec = p.svec && reinterpret_cast<uintptr_t>(sc) % (2 * p.ks) == 0;
#define KQ_SKINNY_SV(LDS_, HL_, M1_, REM_)                                                      \
  do {                                                                                          \
    if (svec)                                                                                   \
      launch_skinny_ks<BITS, LDS_, HL_, true, M1_, REM_>(p, grid, block, shm, st, x, ldx, m, k, \
                                                         xvec, wq, sc, row_bytes, ng, xa, xexp, \
                                                         bias, y, ldy, n, argp);                \
    else                                                                                        \
      launch_skinny_ks<BITS, LDS_, HL_, false, M1_, REM_>(p, grid, block, shm, st, x, ldx, m,   \
                                                          k, xvec, wq, sc, row_bytes, ng, xa,   \
                                                          xexp, bias, y, ldy, n, argp);         \
  } while (0)
  // Do the pre-loads (one batch of KS units at M = 1, else 4 entries per
  // lane over all rows) cover every activation entry of every wave?  The
  // single-row instances are used for INT4 (measured: INT8 runs as fast or
  // faster through the general ones).
  constexpr int kTpu = BITS == 4 ? 4 : 2;
  constexpr int64_t kUnitCols = BITS == 4 ? 128 : 64;
  const int pre1 = std::min(4, std::max(1, p.ks * kTpu / 16));
  // Instances without the remainder block need every entry pre-loadable:
  // aligned x and no K tail inside the last unit (an INT4 K that is not a
  // multiple of 128 leaves tail entries that must be staged as zeros).
  const bool aligned = xvec && k == p.nunits * kUnitCols;
  const bool one_row = BITS == 4 && aligned && m == 1 && p.per_wave * kTpu <= 16 * pre1;
  // (lane mapping: skinny_lanes_per_row(m) lanes per row, 4 pre-load slots each)
  const bool covered = aligned && p.per_wave * kTpu <= skinny_lanes_per_row((int)m);
  if (p.a_lds) {
    if constexpr (BITS == 4) {
      if (p.hl && one_row) {
        KQ_SKINNY_SV(true, true, true, false);
        return kq_check_launch("kq_linear_int4 (skinny)");
      }
    }
    if (p.hl && covered) KQ_SKINNY_SV(true, true, false, false);
    else if (p.hl) KQ_SKINNY_SV(true, true, false, true);
    else KQ_SKINNY_SV(true, false, false, true);
  } else {
    if (p.hl) KQ_SKINNY_SV(false, true, false, false);
    else KQ_SKINNY_SV(false, false, false, false);
  }
#undef KQ_SKINNY_SV
  if (p.ksplit > 1) {
    const bool vec = n % 4 == 0 && ldy_out % 4 == 0 && reinterpret_cast<uintptr_t>(y_out) % 16 == 0 &&
                     (bias_out == nullptr || reinterpret_cast<uintptr_t>(bias_out) % 16 == 0);
    const int64_t items = vec ? m * n / 4 : m * n;
    const unsigned rg = (unsigned)std::min<int64_t>((items + 255) / 256, 8192);
    // BITS = 4 instance: sums only (the slices applied any INT8 row scale)
    if (vec) splitk_reduce_kernel<4, true><<<rg, 256, 0, st>>>(y, (int)p.ksplit, m, n, nullptr, 0, nullptr, bias_out, y_out, ldy_out);
    else splitk_reduce_kernel<4, false><<<rg, 256, 0, st>>>(y, (int)p.ksplit, m, n, nullptr, 0, nullptr, bias_out, y_out, ldy_out);
  }
  return kq_check_launch(BITS == 4 ? "kq_linear_int4 (skinny)" : "kq_linear_int8 (skinny)");
}

template <int BITS, int MTW, int NTW, int WN = kGemmWN>
void launch_gemm_t(const Plan& p, const half8_t* planes, const int* rexp, int64_t m,
                   const uint8_t* wq, const uint16_t* sc, int64_t row_bytes, int64_t ng,
                   const float* bias, float* y, int64_t ldy, int64_t n, float* part, hipStream_t st) {
  const unsigned blocks = (unsigned)(p.tiles_m * p.tiles_n * p.splits);
  gemm_kernel<BITS, MTW, NTW, WN><<<blocks, 64 * WN, 0, st>>>(
      planes, p.mpad, m, wq, sc, row_bytes, ng, p.nstages, p.spz, (int)p.tiles_m, (int)p.tiles_n,
      p.gm, rexp, bias, y, ldy, n, part);
}

template <int BITS>
int launch_gemm(const Plan& p, const float* x, int64_t ldx, int64_t m, int64_t k,
                const uint8_t* wq, const uint16_t* sc, int64_t row_bytes, int64_t ng,
                const float* bias, float* y, int64_t ldy, int64_t n, void* ws, hipStream_t st) {
  half8_t* planes = static_cast<half8_t*>(ws);
  const GemmWs lay = gemm_ws_layout(p);
  int* rexp = reinterpret_cast<int*>(static_cast<char*>(ws) + lay.rexp_off);
  // One workgroup per (padded) row: the row's scale, then its operand planes.
  stage_rows_kernel<BITS, true, false><<<(unsigned)p.mpad, 256, 0, st>>>(
      x, ldx, (int)m, k, (int)(4 * p.nstages), 0, p.mpad, x_vectorizable(x, ldx, k), planes, rexp);
  float* part = p.splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + lay.part_off) : nullptr;
  if (p.wspec) {
    const unsigned blocks = (unsigned)(p.tiles_m * p.tiles_n * p.splits);
#define KQ_WS(D_, NC_, DW_)                                                                     \
  gemm_ws_kernel<BITS, D_, NC_, DW_><<<blocks, 64 * (NC_ + (DW_ > 0 ? 2 : 1)), 0, st>>>(        \
      planes, p.mpad, m, wq, sc, row_bytes, ng, p.nstages, p.spz, (int)p.tiles_m,               \
      (int)p.tiles_n, p.gm, rexp, bias, y, ldy, n, part)
    if constexpr (BITS == 4) {
      if (p.wsdw) KQ_WS(2, kWsNC, 5);
      else if (p.wsnc == kWsWideNC) KQ_WS(2, kWsWideNC, 0);
      else KQ_WS(3, kWsNC, 0);
    } else {
      if (p.wsdw) KQ_WS(2, kWsNC, 3);
      else KQ_WS(2, kWsNC, 0);
    }
#undef KQ_WS
  } else if (p.mtw == 2) {
    if (p.ntw == 2) launch_gemm_t<BITS, 2, 2>(p, planes, rexp, m, wq, sc, row_bytes, ng, bias, y, ldy, n, part, st);
    else if (p.wn == kGemmWideWN8) launch_gemm_t<BITS, 2, 4, kGemmWideWN8>(p, planes, rexp, m, wq, sc, row_bytes, ng, bias, y, ldy, n, part, st);
    else launch_gemm_t<BITS, 2, 4>(p, planes, rexp, m, wq, sc, row_bytes, ng, bias, y, ldy, n, part, st);
  } else {
    if (p.ntw == 2) launch_gemm_t<BITS, 4, 2>(p, planes, rexp, m, wq, sc, row_bytes, ng, bias, y, ldy, n, part, st);
    else launch_gemm_t<BITS, 4, 4>(p, planes, rexp, m, wq, sc, row_bytes, ng, bias, y, ldy, n, part, st);
  }
  if (part) {
    const bool vec = n % 4 == 0 && ldy % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                     (bias == nullptr || reinterpret_cast<uintptr_t>(bias) % 16 == 0);
    const int64_t items = vec ? m * n / 4 : m * n;
    const unsigned rg = (unsigned)std::min<int64_t>((items + 255) / 256, 8192);
    if (vec) splitk_reduce_kernel<BITS, true><<<rg, 256, 0, st>>>(part, (int)p.splits, m, n, rexp, 0, sc, bias, y, ldy);
    else splitk_reduce_kernel<BITS, false><<<rg, 256, 0, st>>>(part, (int)p.splits, m, n, rexp, 0, sc, bias, y, ldy);
  }
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

// Workspace of the linear + greedy-argmax entry points: the linear's own
// workspace, then the per-row partials, then (GEMM / generic paths) a logits
// buffer used when the caller passes none.
struct ArgLayout {
  int64_t parts = 0;
  size_t part_off = 0, logit_off = 0, total = 0;
};


ArgLayout arg_layout(const Plan& p, int64_t m, int64_t n) {
  ArgLayout a;
  const bool skinny = p.path == Path::Skinny;
  a.parts = skinny ? (n + 16 * p.nt - 1) / (16 * p.nt) * p.nt : (n + kArgChunk - 1) / kArgChunk;
  a.part_off = align256(p.ws);
  a.logit_off = align256(a.part_off + (size_t)(m * a.parts) * sizeof(int2));
  a.total = a.logit_off + (skinny ? 0 : (size_t)(m * n) * sizeof(float));
  return a;
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
  if (scheme == 8) return make_plan(8, m, n, k, 0, k, false, true).ws;
  if (group_size <= 0) return 0;
  const int64_t kp = (k + group_size - 1) / group_size * group_size;
  return make_plan(4, m, n, k, group_size, kp, false, true).ws;
}

extern "C" int kq_linear_int8(const float* x, int64_t m, int64_t ldx, const int8_t* payload,
                              const uint16_t* scales, const float* bias, float* y, int64_t ldy,
                              int64_t n, int64_t k, void* ws, size_t ws_bytes,
                              kq_stream_t stream) {
  if (int s = check_linear_args(x, m, ldx, payload, scales, y, ldy, n, k)) return s;
  const Plan p = make_plan(8, m, n, k, 0, k, false, true);
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
  const Plan p = make_plan(4, m, n, k, g, kp, false, true);
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

// ---------------------------------------------------------------------------
// Quantized linear + greedy argmax (the lm_head of engine/model.py:151, read
// by :187,:200): tokens[r] = first index of the maximum of row r's logits.
// ---------------------------------------------------------------------------
namespace {

template <int BITS>
int linear_argmax(const Plan& p, const float* x, int64_t m, int64_t ldx, const uint8_t* wq,
                  const uint16_t* sc, int64_t row_bytes, int64_t g, int64_t ng, const float* bias,
                  float* logits, int64_t ldl, int64_t n, int64_t k, int64_t* tokens, void* ws,
                  size_t ws_bytes, hipStream_t st) {
  const ArgLayout a = arg_layout(p, m, n);
  if (ws == nullptr || ws_bytes < a.total)
    return kq_set_error(KQ_ERR_WORKSPACE, "workspace missing or smaller than kq_linear_argmax_workspace_bytes()");
  char* w = static_cast<char*>(ws);
  int2* argp = reinterpret_cast<int2*>(w + a.part_off);
  int s;
  if (p.path == Path::Skinny) {
    s = launch_skinny<BITS>(p, x, ldx, m, k, wq, sc, row_bytes, ng, bias, logits, ldl, n, w, st, argp);
  } else {
    float* y = logits ? logits : reinterpret_cast<float*>(w + a.logit_off);
    const int64_t ldy = logits ? ldl : n;
    if (p.path == Path::Gemm) s = launch_gemm<BITS>(p, x, ldx, m, k, wq, sc, row_bytes, ng, bias, y, ldy, n, w, st);
    else s = launch_generic<BITS>(x, ldx, m, wq, sc, row_bytes, g, ng, bias, y, ldy, n, k, st);
    if (s == KQ_OK) argmax_partial_kernel<<<dim3((unsigned)a.parts, (unsigned)m), 256, 0, st>>>(y, ldy, n, argp);
  }
  if (s != KQ_OK) return s;
  argmax_final_kernel<<<(unsigned)m, 1024, 0, st>>>(argp, a.parts, tokens);
  return kq_check_launch(BITS == 4 ? "kq_linear_argmax_int4" : "kq_linear_argmax_int8");
}

int check_argmax_args(const float* x, int64_t m, int64_t ldx, const void* wq, const void* sc,
                      const float* logits, int64_t ldl, int64_t n, int64_t k, const int64_t* tokens) {
  KQ_REQUIRE(x != nullptr && wq != nullptr && sc != nullptr && tokens != nullptr, "null pointer argument");
  KQ_REQUIRE(m > 0 && n > 0 && k > 0, "empty linear");
  KQ_REQUIRE(m <= 65535, "more than 65535 rows");
  KQ_REQUIRE(n <= 0x7fffffff, "out_features beyond int32 indices");
  KQ_REQUIRE(ldx >= k, "ldx smaller than in_features");
  KQ_REQUIRE(logits == nullptr || ldl >= n, "ldl smaller than out_features");
  return KQ_OK;
}

}  // namespace

extern "C" size_t kq_linear_argmax_workspace_bytes(int scheme, int64_t m, int64_t n, int64_t k,
                                                   int64_t group_size) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  if (scheme == 8) return arg_layout(make_plan(8, m, n, k, 0, k), m, n).total;
  if (group_size <= 0) return 0;
  const int64_t kp = (k + group_size - 1) / group_size * group_size;
  return arg_layout(make_plan(4, m, n, k, group_size, kp), m, n).total;
}

extern "C" int kq_linear_argmax_int8(const float* x, int64_t m, int64_t ldx, const int8_t* payload,
                                     const uint16_t* scales, const float* bias, float* logits,
                                     int64_t ldl, int64_t n, int64_t k, int64_t* tokens, void* ws,
                                     size_t ws_bytes, kq_stream_t stream) {
  if (int s = check_argmax_args(x, m, ldx, payload, scales, logits, ldl, n, k, tokens)) return s;
  const Plan p = make_plan(8, m, n, k, 0, k);
  return linear_argmax<8>(p, x, m, ldx, reinterpret_cast<const uint8_t*>(payload), scales, k, 1, 1,
                          bias, logits, ldl, n, k, tokens, ws, ws_bytes, kq_stream(stream));
}

extern "C" int kq_linear_argmax_int4(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                                     const uint16_t* scales, int64_t g, int64_t kp, const float* bias,
                                     float* logits, int64_t ldl, int64_t n, int64_t k, int64_t* tokens,
                                     void* ws, size_t ws_bytes, kq_stream_t stream) {
  if (int s = check_argmax_args(x, m, ldx, payload, scales, logits, ldl, n, k, tokens)) return s;
  KQ_REQUIRE(g > 0 && g % 2 == 0, "group_size must be a positive even integer");
  KQ_REQUIRE(kp % g == 0 && kp >= k && kp - k < g, "inconsistent in_features_padded");
  const Plan p = make_plan(4, m, n, k, g, kp);
  return linear_argmax<4>(p, x, m, ldx, payload, scales, kp / 2, g, kp / g, bias, logits, ldl, n, k,
                          tokens, ws, ws_bytes, kq_stream(stream));
}

// ---------------------------------------------------------------------------
// Fused gate / up projection with the SiLU gate: act = silu(x Wg^T + bg) *
// (x Wu^T + bu), the MLP input of HF Llama / Qwen2 (down_proj(act_fn(
// gate_proj(x)) * up_proj(x))), which Kshipra runs inside layer.mlp
// (engine/model.py:147) as two QuantizedLinear calls and two elementwise ops.  The packed
// weight (and scales, bias) interleave the two by 16-row tiles: rows
// 32 b .. 32 b + 15 are gate rows 16 b .. 16 b + 15, the next 16 the same up
// rows.  Skinny path: one gate / up tile pair per wave, silu * up in the
// epilogue.  Other paths: the interleaved product goes to the workspace and
// silu_mul_pairs_kernel combines it.
// ---------------------------------------------------------------------------
namespace {

__global__ __launch_bounds__(256) void silu_mul_pairs_kernel(const float* __restrict__ yi, int64_t m,
                                                             int64_t nh, float* __restrict__ act,
                                                             int64_t lda) {
  const int64_t total = m * nh;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / nh, j = e - r * nh;
    const int64_t src = r * 2 * nh + (j >> 4) * 32 + (j & 15);
    const float g = yi[src], u = yi[src + 16];
    act[r * lda + j] = g / (1.0f + expf(-g)) * u;
  }
}

size_t silu_mul_ws(const Plan& p, int64_t m, int64_t nh) {
  return p.path == Path::Skinny ? p.ws : align256(p.ws) + (size_t)(m * 2 * nh) * sizeof(float);
}

int check_silu_args(const float* x, int64_t m, int64_t ldx, const void* wq, const void* sc,
                    const float* act, int64_t lda, int64_t nh, int64_t k) {
  KQ_REQUIRE(x != nullptr && wq != nullptr && sc != nullptr && act != nullptr, "null pointer argument");
  KQ_REQUIRE(m > 0 && nh > 0 && k > 0, "empty linear");
  KQ_REQUIRE(nh % 16 == 0, "gate / up out_features must be a multiple of 16 (16-row tile pairs)");
  KQ_REQUIRE(ldx >= k, "ldx smaller than in_features");
  KQ_REQUIRE(lda >= nh, "ldact smaller than out_features");
  return KQ_OK;
}

template <int BITS>
int linear_silu_mul(const Plan& p, const float* x, int64_t m, int64_t ldx, const uint8_t* wq,
                    const uint16_t* sc, int64_t row_bytes, int64_t g, int64_t ng, const float* bias,
                    float* act, int64_t lda, int64_t nh, int64_t k, void* ws, size_t ws_bytes,
                    hipStream_t st) {
  if (ws_bytes < silu_mul_ws(p, m, nh) || (silu_mul_ws(p, m, nh) > 0 && ws == nullptr))
    return kq_set_error(KQ_ERR_WORKSPACE, "workspace missing or smaller than kq_linear_silu_mul_workspace_bytes()");
  const int64_t n = 2 * nh;
  if (p.path == Path::Skinny)
    return launch_skinny<BITS>(p, x, ldx, m, k, wq, sc, row_bytes, ng, bias, act, lda, n, ws, st);
  float* yi = reinterpret_cast<float*>(static_cast<char*>(ws) + align256(p.ws));
  int s;
  if (p.path == Path::Gemm) s = launch_gemm<BITS>(p, x, ldx, m, k, wq, sc, row_bytes, ng, bias, yi, n, n, ws, st);
  else s = launch_generic<BITS>(x, ldx, m, wq, sc, row_bytes, g, ng, bias, yi, n, n, k, st);
  if (s != KQ_OK) return s;
  const unsigned blocks = (unsigned)std::min<int64_t>((m * nh + 255) / 256, 8192);
  silu_mul_pairs_kernel<<<blocks, 256, 0, st>>>(yi, m, nh, act, lda);
  return kq_check_launch(BITS == 4 ? "kq_linear_silu_mul_int4" : "kq_linear_silu_mul_int8");
}

}  // namespace

extern "C" size_t kq_linear_silu_mul_workspace_bytes(int scheme, int64_t m, int64_t nh, int64_t k,
                                                     int64_t group_size) {
  if (m <= 0 || nh <= 0 || k <= 0) return 0;
  if (scheme == 8) return silu_mul_ws(make_plan(8, m, 2 * nh, k, 0, k, true), m, nh);
  if (group_size <= 0) return 0;
  const int64_t kp = (k + group_size - 1) / group_size * group_size;
  return silu_mul_ws(make_plan(4, m, 2 * nh, k, group_size, kp, true), m, nh);
}

extern "C" int kq_linear_silu_mul_int8(const float* x, int64_t m, int64_t ldx, const int8_t* payload,
                                       const uint16_t* scales, const float* bias, float* act,
                                       int64_t ldact, int64_t nh, int64_t k, void* ws,
                                       size_t ws_bytes, kq_stream_t stream) {
  if (int s = check_silu_args(x, m, ldx, payload, scales, act, ldact, nh, k)) return s;
  const Plan p = make_plan(8, m, 2 * nh, k, 0, k, true);
  return linear_silu_mul<8>(p, x, m, ldx, reinterpret_cast<const uint8_t*>(payload), scales, k, 1, 1,
                            bias, act, ldact, nh, k, ws, ws_bytes, kq_stream(stream));
}

extern "C" int kq_linear_silu_mul_int4(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                                       const uint16_t* scales, int64_t g, int64_t kp,
                                       const float* bias, float* act, int64_t ldact, int64_t nh,
                                       int64_t k, void* ws, size_t ws_bytes, kq_stream_t stream) {
  if (int s = check_silu_args(x, m, ldx, payload, scales, act, ldact, nh, k)) return s;
  KQ_REQUIRE(g > 0 && g % 2 == 0, "group_size must be a positive even integer");
  KQ_REQUIRE(kp % g == 0 && kp >= k && kp - k < g, "inconsistent in_features_padded");
  const Plan p = make_plan(4, m, 2 * nh, k, g, kp, true);
  return linear_silu_mul<4>(p, x, m, ldx, payload, scales, kp / 2, g, kp / g, bias, act, ldact, nh, k,
                            ws, ws_bytes, kq_stream(stream));
}
