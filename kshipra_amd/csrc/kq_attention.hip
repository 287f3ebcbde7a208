// Paged K/V write and chunked (prefix + chunk) attention over the block pool,
// fp32, for gfx950.
//
//  * kq_paged_kv_write_f32 -- the K/V store of KshipraModel.forward
//    (engine/model.py:124-129): token t's K and V rows of every KV head go to
//    pool[slot // B, layer, 0 / 1, :, slot % B, :], slot = slot_mapping[t].
//    One thread moves 4 floats; HBM-bound, 2 x (read + write) per element.
//  * kq_chunked_attention_f32 -- chunked_attention (engine/chunked_prefill.py:
//    93-140): query i of the chunk (position prefix_len + i) attends to every
//    key at position <= its own, read in place from the pool through the block
//    table, with GQA (query head h reads KV head h / g) and the online softmax.
//
// Attention work decomposition.  Rows of one KV head are (query, head-in-group)
// pairs, row = c * g + hh, so a 16-row tile spans 16 / g consecutive queries of
// all g heads sharing the K / V stream.  One wave owns (KV head, 16-row tile,
// key split) and walks its keys 16 at a time with fp32 MFMA 16x16x4:
//
//   S^T[key][row] = sum_d K[key][d] Q[row][d]          (D / 4 MFMAs)
//   O^T[d][row]  += sum_key V[key][d] P[row][key]       (D / 4 MFMAs)
//
// Computing S^T (keys on the MFMA's row axis) leaves lane l holding row l % 16
// and keys 4 (l / 16) + r in its 4 accumulators -- exactly the B operand
// (P^T, k index l / 16) of the second product, so P never moves between
// lanes.  Both reductions run in a permuted order chosen so every lane reads
// contiguous memory: in the first product lane group q = l / 16 covers d in
// [q D/4, (q+1) D/4) (D/16 float4 loads along its key's row), in the second
// lane l % 16 = j covers d = (D/16) j + db, db = 0 .. D/16-1 (D/64 float4
// loads per key).  (Spreading each load instruction over contiguous runs of
// several lanes instead measured slower.)  Row statistics (running max m,
// sum l) live in the lanes of their row;
// one row's 16 scores are spread over lane groups, so the row max and sum take
// two cross-lane steps.  Scores are in log2 units (Q is pre-scaled by
// log2(e) / sqrt(D)) and exponentials are exp2.
//
// Splits: when KV heads x row tiles gives too few waves to fill the GPU
// (decode, short chunks) the key range is split; each split writes its
// unnormalised (m, l, acc) to the workspace and a second kernel merges them.
#include <algorithm>
#include <cmath>

#include "kq_common.hpp"

namespace {

constexpr int kAttnWavesPerBlock = 4;
constexpr int64_t kAttnTargetWaves = 2048;     // 8 waves per CU on 256 CUs
constexpr int64_t kAttnSplitBelow = 512;       // split keys only below this many row-tile waves
constexpr int64_t kAttnMinTilesPerSplit = 1;
constexpr int64_t kAttnMaxSplits = 256;

struct AttnArgs {
  const float* q;
  const float* kp;
  const float* vp;
  const int32_t* table;
  float* out;
  float* ws_acc;   // [splits][rows_total][D]
  float* ws_ml;    // [splits][rows_total][2]
  int64_t q_ld_head, q_ld_tok;
  int64_t o_ld_head, o_ld_tok;
  int64_t p_ld_blk, p_ld_head, p_ld_off;
  int num_blocks, block_size;
  int group, chunk, prefix, total;
  int rowtiles, splits, split_keys, items, rows_total;
  float qscale;
};

struct AttnPlan {
  int64_t rowtiles, splits, split_keys, items;
};

AttnPlan attn_plan(int64_t hq, int64_t hkv, int64_t chunk, int64_t prefix) {
  AttnPlan p{};
  const int64_t g = hq / hkv;
  p.rowtiles = (g * chunk + 15) / 16;
  const int64_t ntiles = (prefix + chunk + 15) / 16;
  const int64_t base = hkv * p.rowtiles;
  // Row tiles alone fill the GPU from kAttnSplitBelow waves on (measured:
  // the shared-tile kernel at 1024 waves beats 2 splits of the per-wave one
  // by 18 %); decode and short chunks split their keys up to ~2048 waves.
  int64_t splits = 1;
  if (base < kAttnSplitBelow) {
    splits = (kAttnTargetWaves + base - 1) / base;
    splits = std::min(splits, (ntiles + kAttnMinTilesPerSplit - 1) / kAttnMinTilesPerSplit);
    splits = std::min(std::max<int64_t>(splits, 1), kAttnMaxSplits);
  }
  const int64_t tiles_per_split = (ntiles + splits - 1) / splits;
  p.splits = (ntiles + tiles_per_split - 1) / tiles_per_split;   // no empty tail split
  p.split_keys = tiles_per_split * 16;
  p.items = base * p.splits;
  return p;
}

__device__ __forceinline__ floatx4 ld4(const float* p) {
  return *reinterpret_cast<const floatx4*>(p);
}

// Pool row (block, head, offset) of key position pos, pos < total.
__device__ __forceinline__ const float* key_row(const float* pool, const AttnArgs& a, int kvh,
                                                int pos) {
  const int j = pos / a.block_size;
  unsigned blk = (unsigned)a.table[j];
  blk = blk < (unsigned)a.num_blocks ? blk : (unsigned)(a.num_blocks - 1);
  return pool + (int64_t)blk * a.p_ld_blk + (int64_t)kvh * a.p_ld_head +
         (int64_t)(pos - j * a.block_size) * a.p_ld_off;
}

// One 16-key tile of the online softmax for the 16 rows of a wave (lane
// (j16, grp) = row j16; kf / vf: its K / V operands, qv: its pre-scaled Q):
// S^T = K Q^T, causal mask key > qpos, running max / sum update, O^T += V^T P^T.
template <int D>
__device__ __forceinline__ void attn_tile(const float (&kf)[D / 4], const floatx4 (&vf)[4][D / 64],
                                          const float (&qv)[D / 4], int kt0, int qpos, int grp,
                                          float& m, float& l, floatx4 (&acc)[D / 16]) {
  constexpr int DQ = D / 4, DB = D / 16;
  floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < DQ; ++i) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[i], qv[i], s, 0, 0, 0);
  // Causal mask (covers positions past the sequence: qpos <= total - 1).
  float sv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) sv[r] = (kt0 + 4 * grp + r > qpos) ? -__builtin_inff() : s[r];
  float mx = __builtin_fmaxf(__builtin_fmaxf(sv[0], sv[1]), __builtin_fmaxf(sv[2], sv[3]));
  mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float mnew = __builtin_fmaxf(m, mx);
  const float msafe = mnew == -__builtin_inff() ? 0.f : mnew;
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(sv[r] - msafe);
  const float corr = __builtin_amdgcn_exp2f(m - msafe);
  float ps = (p[0] + p[1]) + (p[2] + p[3]);
  ps += __shfl_xor(ps, 16, 64);
  ps += __shfl_xor(ps, 32, 64);
  l = l * corr + ps;
  m = mnew;
#pragma unroll
  for (int i = 0; i < DB; ++i) acc[i] *= corr;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int i = 0; i < DB; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[r][i / 4][i % 4], p[r], acc[i], 0, 0, 0);
}

// Occupancy 3 (<= 168 registers per lane): measured faster than 2.
template <int D, bool BLK16>
__global__ __launch_bounds__(64 * kAttnWavesPerBlock, 3) void chunked_attention_kernel(const AttnArgs a) {
  constexpr int DQ = D / 4;    // d per lane group in S^T = K Q^T
  constexpr int DB = D / 16;   // d-blocks of O^T (floats per lane per key in V)
  const int lane = threadIdx.x & 63;

  // XCD-aware order: blocks b, b + 8, ... share an XCD (and its L2); give each
  // XCD a contiguous range of items (same KV head, neighbouring row tiles).
  int b = blockIdx.x;
  if ((gridDim.x & 7) == 0) b = (b & 7) * (gridDim.x >> 3) + (b >> 3);
  int item = b * kAttnWavesPerBlock + (threadIdx.x >> 6);
  if (item >= a.items) return;
  const int split = item % a.splits;
  item /= a.splits;
  const int rt = item % a.rowtiles;
  const int kvh = item / a.rowtiles;

  const int g = a.group;
  const int rows = g * a.chunk;
  const int j16 = lane & 15, grp = lane >> 4;
  const int rho = rt * 16 + j16;
  const bool rvalid = rho < rows;
  const int c = rvalid ? rho / g : 0;
  const int head = kvh * g + (rvalid ? rho - c * g : 0);
  const int qpos = a.prefix + c;

  float qv[DQ];
  {
    const float* qp = a.q + (int64_t)head * a.q_ld_head + (int64_t)c * a.q_ld_tok + DQ * grp;
#pragma unroll
    for (int i = 0; i < DQ / 4; ++i) {
      floatx4 t = rvalid ? ld4(qp + 4 * i) : floatx4{0.f, 0.f, 0.f, 0.f};
      qv[4 * i + 0] = t[0] * a.qscale;
      qv[4 * i + 1] = t[1] * a.qscale;
      qv[4 * i + 2] = t[2] * a.qscale;
      qv[4 * i + 3] = t[3] * a.qscale;
    }
  }

  // Keys this wave reads: its split's range, cut at the last position any
  // row of the tile may see.
  const int rlast = min(rt * 16 + 15, rows - 1);
  const int kend = min(a.total, a.prefix + rlast / g + 1);
  const int kbeg = split * a.split_keys;
  const int kstop = min(kbeg + a.split_keys, kend);

  float m = -__builtin_inff(), l = 0.f;
  floatx4 acc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Tile loads: K row of key kt0 + j16 (from d = DQ grp), V rows of keys
  // kt0 + 4 grp + r (from d = DB j16).  Positions are clamped to the wave's
  // last key, kstop - 1: inside a tile, positions >= kstop occur only when
  // kstop is the causal / sequence end, where they are masked.  (Prefetching
  // tile t + 1 during tile t measured slower: it doubles the K / V registers
  // and drops occupancy from 3 to 2.)
  const int lastk = kstop - 1;
  struct Tile {
    float k[DQ];
    floatx4 v[4][DB / 4];
  };
  auto load = [&](Tile& t, int kt0) {
    if constexpr (BLK16) {
      // B % 16 == 0: the (clamped) keys of the tile share one block.
      const int j = min(kt0, lastk) / a.block_size;
      unsigned blk = (unsigned)a.table[j];
      blk = blk < (unsigned)a.num_blocks ? blk : (unsigned)(a.num_blocks - 1);
      const int64_t hb = (int64_t)blk * a.p_ld_blk + (int64_t)kvh * a.p_ld_head;
      const int o0 = j * a.block_size;
      const float* kr = a.kp + hb + (int64_t)(min(kt0 + j16, lastk) - o0) * a.p_ld_off + DQ * grp;
#pragma unroll
      for (int i = 0; i < DQ / 4; ++i) {
        const floatx4 x = ld4(kr + 4 * i);
        t.k[4 * i + 0] = x[0]; t.k[4 * i + 1] = x[1]; t.k[4 * i + 2] = x[2]; t.k[4 * i + 3] = x[3];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vr = a.vp + hb + (int64_t)(min(kt0 + 4 * grp + r, lastk) - o0) * a.p_ld_off + DB * j16;
#pragma unroll
        for (int i = 0; i < DB / 4; ++i) t.v[r][i] = ld4(vr + 4 * i);
      }
    } else {
      const float* kr = key_row(a.kp, a, kvh, min(kt0 + j16, lastk)) + DQ * grp;
#pragma unroll
      for (int i = 0; i < DQ / 4; ++i) {
        const floatx4 x = ld4(kr + 4 * i);
        t.k[4 * i + 0] = x[0]; t.k[4 * i + 1] = x[1]; t.k[4 * i + 2] = x[2]; t.k[4 * i + 3] = x[3];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vr = key_row(a.vp, a, kvh, min(kt0 + 4 * grp + r, lastk)) + DB * j16;
#pragma unroll
        for (int i = 0; i < DB / 4; ++i) t.v[r][i] = ld4(vr + 4 * i);
      }
    }
  };
  for (int kt0 = kbeg; kt0 < kstop; kt0 += 16) {
    Tile t;
    load(t, kt0);
    attn_tile<D>(t.k, t.v, qv, kt0, qpos, grp, m, l, acc);
  }

  if (!rvalid) return;
  // Lane holds O^T[4 grp + r'][row] of d-block i: d = DB (4 grp + r') + i.
  if (a.splits == 1) {
    const float inv = 1.f / l;
    float* op = a.out + (int64_t)head * a.o_ld_head + (int64_t)c * a.o_ld_tok;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = op + DB * (4 * grp + r);
#pragma unroll
      for (int i = 0; i < DB / 4; ++i) {
        floatx4 t;
        t[0] = acc[4 * i + 0][r] * inv; t[1] = acc[4 * i + 1][r] * inv;
        t[2] = acc[4 * i + 2][r] * inv; t[3] = acc[4 * i + 3][r] * inv;
        *reinterpret_cast<floatx4*>(dst + 4 * i) = t;
      }
    }
  } else {
    const int64_t rowg = (int64_t)split * a.rows_total + (int64_t)kvh * rows + rho;
    float* wp = a.ws_acc + rowg * D;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = wp + DB * (4 * grp + r);
#pragma unroll
      for (int i = 0; i < DB / 4; ++i) {
        floatx4 t;
        t[0] = acc[4 * i + 0][r]; t[1] = acc[4 * i + 1][r];
        t[2] = acc[4 * i + 2][r]; t[3] = acc[4 * i + 3][r];
        *reinterpret_cast<floatx4*>(dst + 4 * i) = t;
      }
    }
    if (grp == 0) {
      a.ws_ml[2 * rowg + 0] = m;
      a.ws_ml[2 * rowg + 1] = l;
    }
  }
}

// Unsplit walks (prefill chunks): the 4 waves of a workgroup own 4
// consecutive row tiles of one KV head and walk the same keys, so each
// 16-key K / V tile is loaded once per workgroup -- all 256 threads, 4 KB
// of it each (16 threads per key row) -- into a double-buffered LDS tile and
// read from there by every wave (4x less L2 -> CU traffic than each wave
// streaming its own copy).  The workgroup walks up to the last causal
// position of its last row tile; a wave skips the math of tiles past its
// own.  Rows are padded by D + 4 floats so the 16 rows one LDS read
// instruction touches fall in different banks.
template <int D>
struct KvTileLds {
  float k[16][D + 4];
  float v[16][D + 4];
};

template <int D, bool BLK16>
__global__ __launch_bounds__(64 * kAttnWavesPerBlock, 3) void chunked_attention_shared_kernel(const AttnArgs a) {
  constexpr int DQ = D / 4, DB = D / 16;
  constexpr int PF = D / 64;   // float4 of a K (and of a V) row per loading thread
  static_assert(kAttnWavesPerBlock == 4, "256 loading threads: 16 per key row");
  __shared__ KvTileLds<D> sm[2];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;

  int b = blockIdx.x;
  if ((gridDim.x & 7) == 0) b = (b & 7) * (gridDim.x >> 3) + (b >> 3);
  const int rtb = (a.rowtiles + kAttnWavesPerBlock - 1) / kAttnWavesPerBlock;
  const int kvh = b / rtb;
  const int rt0 = (b - kvh * rtb) * kAttnWavesPerBlock;
  const int rt = rt0 + w;

  const int g = a.group;
  const int rows = g * a.chunk;
  const int j16 = lane & 15, grp = lane >> 4;
  const int rho = rt * 16 + j16;
  const bool rvalid = rho < rows;
  const int c = rvalid ? rho / g : 0;
  const int head = kvh * g + (rvalid ? rho - c * g : 0);
  const int qpos = a.prefix + c;

  float qv[DQ];
  {
    const float* qp = a.q + (int64_t)head * a.q_ld_head + (int64_t)c * a.q_ld_tok + DQ * grp;
#pragma unroll
    for (int i = 0; i < DQ / 4; ++i) {
      floatx4 t = rvalid ? ld4(qp + 4 * i) : floatx4{0.f, 0.f, 0.f, 0.f};
      qv[4 * i + 0] = t[0] * a.qscale;
      qv[4 * i + 1] = t[1] * a.qscale;
      qv[4 * i + 2] = t[2] * a.qscale;
      qv[4 * i + 3] = t[3] * a.qscale;
    }
  }

  // Keys this wave's rows may see, and those of the workgroup's last row.
  const int kend_w = rt * 16 < rows ? min(a.total, a.prefix + min(rt * 16 + 15, rows - 1) / g + 1) : 0;
  const int rt_last = min(rt0 + kAttnWavesPerBlock - 1, a.rowtiles - 1);
  const int kend = min(a.total, a.prefix + min(rt_last * 16 + 15, rows - 1) / g + 1);
  const int lastk = kend - 1;

  // Loader: thread t moves float4s [t % 16 * PF, +PF) of key row t / 16 of
  // the tile (K and V); positions past the workgroup's keys are clamped to
  // its last key (in bounds; masked or never used).
  const int ck = threadIdx.x >> 4, cp = threadIdx.x & 15;
  floatx4 kr[PF], vr[PF];
  auto gload = [&](int kt0) {
    const int pos = min(kt0 + ck, lastk);
    const float* krow;
    const float* vrow;
    if constexpr (BLK16) {
      const int j = min(kt0, lastk) / a.block_size;
      unsigned blk = (unsigned)a.table[j];
      blk = blk < (unsigned)a.num_blocks ? blk : (unsigned)(a.num_blocks - 1);
      const int64_t off = (int64_t)blk * a.p_ld_blk + (int64_t)kvh * a.p_ld_head +
                          (int64_t)(pos - j * a.block_size) * a.p_ld_off;
      krow = a.kp + off;
      vrow = a.vp + off;
    } else {
      krow = key_row(a.kp, a, kvh, pos);
      vrow = key_row(a.vp, a, kvh, pos);
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      kr[i] = ld4(krow + 4 * (cp * PF + i));
      vr[i] = ld4(vrow + 4 * (cp * PF + i));
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      *reinterpret_cast<floatx4*>(&sm[buf].k[ck][4 * (cp * PF + i)]) = kr[i];
      *reinterpret_cast<floatx4*>(&sm[buf].v[ck][4 * (cp * PF + i)]) = vr[i];
    }
  };

  float m = -__builtin_inff(), l = 0.f;
  floatx4 acc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  gload(0);
  sstore(0);
  __syncthreads();
  int buf = 0;
  for (int kt0 = 0; kt0 < kend; kt0 += 16) {
    const bool more = kt0 + 16 < kend;
    if (more) gload(kt0 + 16);          // next tile in flight during this one's math
    if (kt0 < kend_w) {
      float kf[DQ];
      floatx4 vf[4][DB / 4];
#pragma unroll
      for (int i = 0; i < DQ / 4; ++i) {
        const floatx4 x = *reinterpret_cast<const floatx4*>(&sm[buf].k[j16][DQ * grp + 4 * i]);
        kf[4 * i + 0] = x[0]; kf[4 * i + 1] = x[1]; kf[4 * i + 2] = x[2]; kf[4 * i + 3] = x[3];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < DB / 4; ++i)
          vf[r][i] = *reinterpret_cast<const floatx4*>(&sm[buf].v[4 * grp + r][DB * j16 + 4 * i]);
      attn_tile<D>(kf, vf, qv, kt0, qpos, grp, m, l, acc);
    }
    if (more) sstore(buf ^ 1);          // the other buffer: last read before the previous barrier
    __syncthreads();
    buf ^= 1;
  }

  if (!rvalid) return;
  // Lane holds O^T[4 grp + r'][row] of d-block i: d = DB (4 grp + r') + i.
  const float inv = 1.f / l;
  float* op = a.out + (int64_t)head * a.o_ld_head + (int64_t)c * a.o_ld_tok;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float* dst = op + DB * (4 * grp + r);
#pragma unroll
    for (int i = 0; i < DB / 4; ++i) {
      floatx4 t;
      t[0] = acc[4 * i + 0][r] * inv; t[1] = acc[4 * i + 1][r] * inv;
      t[2] = acc[4 * i + 2][r] * inv; t[3] = acc[4 * i + 3][r] * inv;
      *reinterpret_cast<floatx4*>(dst + 4 * i) = t;
    }
  }
}

// Merges the splits of a row: M = max m_s, out = sum acc_s 2^(m_s - M) /
// sum l_s 2^(m_s - M); a split that saw no visible key has m = -inf, l = 0.
// A workgroup owns COLS float4 columns of one row; thread t takes column
// t % COLS of splits t / COLS + j SG (j < kCombinePerThread), all loaded in
// one round trip.  The row maximum is reduced across the workgroup, then
// the SG partial sums of a column meet by shuffles within each wave (a
// fixed xor tree) and across the 4 waves in LDS.
constexpr int kCombinePerThread = 4;
template <int D, int COLS>
__global__ __launch_bounds__(256) void attention_combine_kernel(const AttnArgs a) {
  constexpr int NV = D / 4;
  constexpr int SG = 256 / COLS;
  static_assert(NV % COLS == 0 && 64 % COLS == 0, "columns");
  __shared__ float red[4];
  __shared__ floatx4 po[4][COLS];
  __shared__ float pl[4][COLS];
  const int t = threadIdx.x, wv = t >> 6;
  const int row = blockIdx.x / (NV / COLS);
  const int v4 = (blockIdx.x % (NV / COLS)) * COLS + t % COLS;
  const int sg = t / COLS;
  float ms[kCombinePerThread], lv[kCombinePerThread];
  floatx4 av[kCombinePerThread];
#pragma unroll
  for (int j = 0; j < kCombinePerThread; j++) {
    const int s = sg + j * SG;
    const bool ok = s < a.splits;
    // past the last split: read split 0 (in bounds) and discard it
    const int64_t rs = (int64_t)(ok ? s : 0) * a.rows_total + row;
    const float m = a.ws_ml[2 * rs], l = a.ws_ml[2 * rs + 1];
    const floatx4 v = ld4(a.ws_acc + rs * D + 4 * v4);
    ms[j] = ok ? m : -__builtin_inff();
    lv[j] = ok ? l : 0.f;
    av[j] = ok ? v : floatx4{0.f, 0.f, 0.f, 0.f};
  }
  float mx = ms[0];
#pragma unroll
  for (int j = 1; j < kCombinePerThread; j++) mx = __builtin_fmaxf(mx, ms[j]);
  mx = wave_max(mx);
  if ((t & 63) == 0) red[wv] = mx;
  __syncthreads();
  mx = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
  const float msafe = mx == -__builtin_inff() ? 0.f : mx;
  floatx4 o = {0.f, 0.f, 0.f, 0.f};
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < kCombinePerThread; j++) {
    const float w = __builtin_amdgcn_exp2f(ms[j] - msafe);
    ls += lv[j] * w;
    o += av[j] * w;
  }
#pragma unroll
  for (int off = COLS; off < 64; off <<= 1) {
    ls += __shfl_xor(ls, off);
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] += __shfl_xor(o[i], off);
  }
  if ((t & 63) < COLS) {
    po[wv][t & 63] = o;
    pl[wv][t & 63] = ls;
  }
  __syncthreads();
  if (t >= COLS) return;
  const floatx4 sum = (po[0][t] + po[1][t]) + (po[2][t] + po[3][t]);
  const float lsum = (pl[0][t] + pl[1][t]) + (pl[2][t] + pl[3][t]);
  const int rows = a.group * a.chunk;
  const int kvh = row / rows, rho = row - kvh * rows;
  const int c = rho / a.group;
  const int head = kvh * a.group + (rho - c * a.group);
  *reinterpret_cast<floatx4*>(a.out + (int64_t)head * a.o_ld_head + (int64_t)c * a.o_ld_tok +
                              4 * v4) = sum * (1.f / lsum);
}

__global__ __launch_bounds__(256) void paged_kv_write_kernel(
    const float* __restrict__ k, const float* __restrict__ v, int tokens, int heads, int d4,
    int64_t s_tok, int64_t s_head, const int64_t* __restrict__ slots, float* __restrict__ kp,
    float* __restrict__ vp, int64_t nslots, int block_size, int64_t p_ld_blk, int64_t p_ld_head,
    int64_t p_ld_off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)tokens * heads * d4) return;
  const int q4 = (int)(i % d4);
  const int64_t th = i / d4;
  const int h = (int)(th % heads);
  const int t = (int)(th / heads);
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= nslots) return;
  const int64_t blk = slot / block_size, off = slot - blk * block_size;
  const int64_t src = (int64_t)t * s_tok + (int64_t)h * s_head + 4 * q4;
  const int64_t dst = blk * p_ld_blk + (int64_t)h * p_ld_head + off * p_ld_off + 4 * q4;
  *reinterpret_cast<floatx4*>(kp + dst) = *reinterpret_cast<const floatx4*>(k + src);
  *reinterpret_cast<floatx4*>(vp + dst) = *reinterpret_cast<const floatx4*>(v + src);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int D>
int launch_attention(const AttnArgs& a, bool blk16, hipStream_t st) {
  if (a.splits == 1) {
    // Unsplit: workgroups of 4 row tiles sharing K / V tiles through LDS.
    const int64_t rtb = (a.rowtiles + kAttnWavesPerBlock - 1) / kAttnWavesPerBlock;
    const int blocks = (int)(rtb * (a.rows_total / (a.group * a.chunk)));
    if (blk16)
      chunked_attention_shared_kernel<D, true><<<blocks, 64 * kAttnWavesPerBlock, 0, st>>>(a);
    else
      chunked_attention_shared_kernel<D, false><<<blocks, 64 * kAttnWavesPerBlock, 0, st>>>(a);
    return kq_check_launch("chunked_attention");
  }
  const int blocks = (a.items + kAttnWavesPerBlock - 1) / kAttnWavesPerBlock;
  if (blk16)
    chunked_attention_kernel<D, true><<<blocks, 64 * kAttnWavesPerBlock, 0, st>>>(a);
  else
    chunked_attention_kernel<D, false><<<blocks, 64 * kAttnWavesPerBlock, 0, st>>>(a);
  if (a.splits > 1) {
    // Few rows with many splits (decode): 4 columns per workgroup, 64 split
    // groups; many rows with few splits: one workgroup per row.  Either way
    // each thread merges at most kCombinePerThread splits.
    static_assert(kAttnMaxSplits <= kCombinePerThread * 64, "combine coverage (4 columns)");
    static_assert(32 <= kCombinePerThread * (256 / (D / 4)), "combine coverage (one row)");
    if (a.splits >= 32)
      attention_combine_kernel<D, 4><<<a.rows_total * (D / 16), 256, 0, st>>>(a);
    else
      attention_combine_kernel<D, D / 4><<<a.rows_total, 256, 0, st>>>(a);
  }
  return kq_check_launch("chunked_attention");
}

}  // namespace

extern "C" size_t kq_chunked_attention_workspace_bytes(int64_t q_heads, int64_t kv_heads,
                                                       int64_t chunk_len, int64_t head_dim,
                                                       int64_t prefix_len) {
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 || chunk_len <= 0 ||
      head_dim <= 0 || prefix_len < 0)
    return 0;
  const AttnPlan p = attn_plan(q_heads, kv_heads, chunk_len, prefix_len);
  if (p.splits <= 1) return 0;
  return (size_t)p.splits * (size_t)(q_heads * chunk_len) * (size_t)(head_dim + 2) * sizeof(float);
}

extern "C" int kq_chunked_attention_f32(
    const float* q, int64_t q_heads, int64_t chunk_len, int64_t head_dim, int64_t q_ld_head,
    int64_t q_ld_tok, const float* k_pool, const float* v_pool, int64_t kv_heads,
    int64_t num_blocks, int64_t block_size, int64_t pool_ld_blk, int64_t pool_ld_head,
    int64_t pool_ld_off, const int32_t* block_table, int64_t table_len, int64_t prefix_len,
    float* out, int64_t out_ld_head, int64_t out_ld_tok, void* workspace,
    size_t workspace_bytes, kq_stream_t stream) {
  KQ_REQUIRE(q_heads > 0 && kv_heads > 0, "head counts must be positive");
  KQ_REQUIRE(q_heads % kv_heads == 0, "GQA requires q_heads % kv_heads == 0");
  KQ_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128");
  KQ_REQUIRE(chunk_len >= 0 && prefix_len >= 0, "chunk_len and prefix_len must be >= 0");
  KQ_REQUIRE(block_size > 0 && num_blocks > 0, "block_size and num_blocks must be positive");
  if (chunk_len == 0) return KQ_OK;
  const int64_t total = prefix_len + chunk_len;
  KQ_REQUIRE(table_len >= (total + block_size - 1) / block_size,
             "block_table shorter than ceil((prefix_len + chunk_len) / block_size)");
  KQ_REQUIRE(total < (int64_t(1) << 30) && q_heads * chunk_len < (int64_t(1) << 30),
             "sequence too long");
  KQ_REQUIRE(q && k_pool && v_pool && block_table && out, "null pointer");
  KQ_REQUIRE(aligned16(q) && aligned16(k_pool) && aligned16(v_pool) && aligned16(out),
             "q, pools and out must be 16-byte aligned");
  KQ_REQUIRE(q_ld_head % 4 == 0 && q_ld_tok % 4 == 0 && out_ld_head % 4 == 0 &&
                 out_ld_tok % 4 == 0 && pool_ld_blk % 4 == 0 && pool_ld_head % 4 == 0 &&
                 pool_ld_off % 4 == 0,
             "strides must be multiples of 4 elements");
  const AttnPlan p = attn_plan(q_heads, kv_heads, chunk_len, prefix_len);
  AttnArgs a{};
  a.q = q; a.kp = k_pool; a.vp = v_pool; a.table = block_table; a.out = out;
  a.q_ld_head = q_ld_head; a.q_ld_tok = q_ld_tok;
  a.o_ld_head = out_ld_head; a.o_ld_tok = out_ld_tok;
  a.p_ld_blk = pool_ld_blk; a.p_ld_head = pool_ld_head; a.p_ld_off = pool_ld_off;
  a.num_blocks = (int)std::min<int64_t>(num_blocks, INT32_MAX);
  a.block_size = (int)block_size;
  a.group = (int)(q_heads / kv_heads);
  a.chunk = (int)chunk_len; a.prefix = (int)prefix_len; a.total = (int)total;
  a.rowtiles = (int)p.rowtiles; a.splits = (int)p.splits; a.split_keys = (int)p.split_keys;
  a.items = (int)p.items; a.rows_total = (int)(q_heads * chunk_len);
  a.qscale = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
  if (p.splits > 1) {
    const size_t need =
        kq_chunked_attention_workspace_bytes(q_heads, kv_heads, chunk_len, head_dim, prefix_len);
    if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
      return kq_set_error(KQ_ERR_WORKSPACE,
                          "workspace missing, misaligned or smaller than "
                          "kq_chunked_attention_workspace_bytes()");
    a.ws_acc = static_cast<float*>(workspace);
    a.ws_ml = a.ws_acc + (size_t)p.splits * a.rows_total * head_dim;
  }
  const bool blk16 = block_size % 16 == 0;
  hipStream_t st = kq_stream(stream);
  return head_dim == 64 ? launch_attention<64>(a, blk16, st) : launch_attention<128>(a, blk16, st);
}

extern "C" int kq_paged_kv_write_f32(const float* k, const float* v, int64_t tokens,
                                     int64_t kv_heads, int64_t head_dim, int64_t src_ld_tok,
                                     int64_t src_ld_head, const int64_t* slot_mapping,
                                     float* k_pool, float* v_pool, int64_t num_blocks,
                                     int64_t block_size, int64_t pool_ld_blk,
                                     int64_t pool_ld_head, int64_t pool_ld_off,
                                     kq_stream_t stream) {
  KQ_REQUIRE(tokens >= 0 && kv_heads > 0 && head_dim > 0, "bad shape");
  KQ_REQUIRE(head_dim % 4 == 0, "head_dim must be a multiple of 4");
  KQ_REQUIRE(num_blocks > 0 && block_size > 0, "num_blocks and block_size must be positive");
  if (tokens == 0) return KQ_OK;
  KQ_REQUIRE(k && v && slot_mapping && k_pool && v_pool, "null pointer");
  KQ_REQUIRE(aligned16(k) && aligned16(v) && aligned16(k_pool) && aligned16(v_pool),
             "k, v and pools must be 16-byte aligned");
  KQ_REQUIRE(src_ld_tok % 4 == 0 && src_ld_head % 4 == 0 && pool_ld_blk % 4 == 0 &&
                 pool_ld_head % 4 == 0 && pool_ld_off % 4 == 0,
             "strides must be multiples of 4 elements");
  const int64_t n = tokens * kv_heads * (head_dim / 4);
  // one thread per 4 floats, 256 per workgroup: the grid must stay below 2^31 workgroups
  KQ_REQUIRE(n < (int64_t(1) << 38) && tokens < INT32_MAX && block_size < INT32_MAX, "too large");
  const int64_t blocks = (n + 255) / 256;
  paged_kv_write_kernel<<<(unsigned)blocks, 256, 0, kq_stream(stream)>>>(
      k, v, (int)tokens, (int)kv_heads, (int)(head_dim / 4), src_ld_tok, src_ld_head,
      slot_mapping, k_pool, v_pool, num_blocks * block_size, (int)block_size, pool_ld_blk,
      pool_ld_head, pool_ld_off);
  return kq_check_launch("paged_kv_write");
}
