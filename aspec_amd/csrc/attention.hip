// DSpark block-sparse attention on gfx950: forward, backward prepare, dQ, dK/dV and finalize.
//
// Masking semantics (direct_cp.py:382-425 / thd_attention.py:77-131, as interval endpoints from
// direct_cp.py:750-900): query row q sees key k iff cb[q] <= k < ce[q] or db[q] <= k < de[q].
// Only tiles listed in the plan are visited; "full" tiles skip the predicate.
//
// One workgroup stacks the G = Hq/Hkv query heads of one KV head (one wave per head) so each K/V
// tile is staged in LDS once for the whole GQA group. Scores are computed transposed
// (S^T = K Q^T) so each lane owns one query row: the softmax statistics are per-lane scalars and
// P^T feeds the P.V MFMA straight from registers.
//
// Tile loops are software pipelined: the global loads of the next tile are in flight in registers
// while the current tile is computed from LDS.
#include "attn_common.h"
#include "plan.h"

namespace aspec {
namespace {

constexpr int kTM = kFwdTileM;          // query rows per wave (one per lane column)
constexpr int kTN = kFwdTileN;          // keys per tile
constexpr int kVtLd = kTN + 4;          // transposed 64-key tile stride (136 B)
constexpr int kQtLd = kBwdTileM + 4;    // transposed 32-row tile stride (72 B)
constexpr int kMaxGroup = 8;
constexpr int kKvWaves = kBwdTileN / 32;
constexpr int kUnitChunkBits = 12;
// Online softmax keeps a stale row maximum until a tile raises it by more than 2^8: exp2 of the
// shifted scores stays <= 256 (exact in fp32, fine in bf16) and O is rescaled only then.
constexpr float kRescaleThreshold = 8.f;

struct AttnArgs {
  const uint16_t* q; int64_t qst, qsh;
  const uint16_t* k; int64_t kst, ksh;
  const uint16_t* v; int64_t vst, vsh;
  const uint16_t* o; int64_t ost, osh;
  const uint16_t* dout; int64_t dost, dosh;
  const int32_t* ends;
  PlanView plan;
  int64_t nq, nk;
  int hq, hkv, group;
  float scale, scale_log2;
  uint16_t* out;       // forward output
  float* lse;          // forward LSE [Hq][Nq]
  const float* lse_in; // backward
  const float* dlse;
  float* ws_delta;     // [Hq][Nq] rowsum(dO*O) - dLSE
  float* ws_lse2;      // [Hq][Nq] LSE * log2(e)
  float* ws_dk;        // [K][Hkv][D] fp32 accumulators of key tiles split over several units
  float* ws_dv;
  uint16_t* dq; int64_t dqst, dqsh;
  uint16_t* dk; int64_t dkst, dksh;
  uint16_t* dv; int64_t dvst, dvsh;
};

// Register-staged tile of ROWS rows x 128 dims, split into 4-row x 8-dim items over NT threads.
// load() issues the global reads of rows [0, valid) of the tile (rows past `valid` are read
// clamped and zeroed: no divergent branches); store() writes the row-major and/or transposed LDS
// copies.
template <int NT, int ROWS>
struct TileLoader {
  static constexpr int kItems = ROWS / 4 * (kHeadDim / 8);
  static constexpr int kPer = (kItems + NT - 1) / NT;
  static constexpr bool kEven = kItems % NT == 0;
  uint4 v[kPer][4];

  __device__ __forceinline__ static bool active(int tid, int p) { return kEven || tid + p * NT < kItems; }
  __device__ __forceinline__ static int row_of(int tid, int p) { return (tid + p * NT) / 16 * 4; }
  __device__ __forceinline__ static int col_of(int tid, int p) { return ((tid + p * NT) % 16) * 8; }

  __device__ __forceinline__ void load(const uint16_t* __restrict__ base, int64_t stride, int valid,
                                       int tid) {
    if (valid >= ROWS) {
#pragma unroll
      for (int p = 0; p < kPer; ++p) {
        if (!active(tid, p)) continue;
        const uint16_t* ptr = base + row_of(tid, p) * stride + col_of(tid, p);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[p][j] = load16(ptr + j * stride);
      }
    } else {
#pragma unroll
      for (int p = 0; p < kPer; ++p) {
        if (!active(tid, p)) continue;
        const int r = row_of(tid, p);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int rr = min(r + j, valid - 1);
          const uint4 x = load16(base + rr * stride + col_of(tid, p));
          v[p][j] = r + j < valid ? x : make_uint4(0, 0, 0, 0);
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* rm, uint16_t* tr, int t_ld, int tid) const {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      if (!active(tid, p)) continue;
      const int r = row_of(tid, p);
      const int col = col_of(tid, p);
      if (rm) {
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(rm + (r + j) * kRowLd + col) = v[p][j];
      }
      if (tr) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          u32x2 w;
          w.x = static_cast<uint32_t>(half_of(v[p][0], e)) | (static_cast<uint32_t>(half_of(v[p][1], e)) << 16);
          w.y = static_cast<uint32_t>(half_of(v[p][2], e)) | (static_cast<uint32_t>(half_of(v[p][3], e)) << 16);
          *reinterpret_cast<u32x2*>(tr + (col + e) * t_ld + r) = w;
        }
      }
    }
  }
};

// Operand fragment of one row: 8 x 16 dims at g*8 of each 16-wide step (rows past the tensor are
// read clamped and zeroed).
__device__ __forceinline__ void load_row_frag(bf16x8 (&frag)[8], const uint16_t* base_valid_row,
                                              bool valid, int g) {
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) {
    const uint4 x = load16(base_valid_row + ds * 16 + g * 8);
    frag[ds] = as_bf16x8(valid ? x : make_uint4(0, 0, 0, 0));
  }
}

// The MFMA chains below load their LDS operands one k-step ahead and fence each step with a
// scheduling barrier: without it the scheduler hoists every LDS read of the tile to the top,
// which overflows the VGPR budget and parks operands in AGPRs.
#define ASPEC_STEP_FENCE() __builtin_amdgcn_sched_barrier(0)

// Two independent 8-step chains: acc0 += A0 x B0, acc1 += A1 x B1 over the 128-dim reduction.
// A rows live in LDS (row-major, `ra0` / `ra1` at this lane's row and g*8); the B operands come
// from registers (`b0`, `b1`) or, when null, from LDS rows `rb0` / `rb1`.
__device__ __forceinline__ void mfma_chains2(f32x16& acc0, f32x16& acc1, const uint16_t* ra0,
                                             const uint16_t* ra1, const bf16x8* b0,
                                             const bf16x8* b1, const uint16_t* rb0,
                                             const uint16_t* rb1) {
  acc0 = f32x16{};
  acc1 = f32x16{};
  uint4 a0 = load16(ra0), a1 = load16(ra1);
  uint4 x0 = b0 ? uint4{} : load16(rb0), x1 = b1 ? uint4{} : load16(rb1);
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) {
    uint4 na0{}, na1{}, nx0{}, nx1{};
    if (ds < 7) {
      na0 = load16(ra0 + (ds + 1) * 16);
      na1 = load16(ra1 + (ds + 1) * 16);
      if (!b0) nx0 = load16(rb0 + (ds + 1) * 16);
      if (!b1) nx1 = load16(rb1 + (ds + 1) * 16);
    }
    acc0 = mfma32(as_bf16x8(a0), b0 ? b0[ds] : as_bf16x8(x0), acc0);
    acc1 = mfma32(as_bf16x8(a1), b1 ? b1[ds] : as_bf16x8(x1), acc1);
    ASPEC_STEP_FENCE();
    a0 = na0;
    a1 = na1;
    x0 = nx0;
    x1 = nx1;
  }
}

// acc[d] += A(d, ks) x B[ks] for d = 0..3 and k-steps ks = 0..KS-1, where A(d, ks) is the
// transposed fragment of the row-major LDS `tile` (rows = the reduction index, 16 per k-step;
// columns d*32 .. +32 = the output rows), read with transpose loads.
template <int KS>
__device__ __forceinline__ void mfma_tr_blocks(f32x16 (&acc)[4], const uint16_t* tile,
                                               const bf16x8 (&b)[KS], int lane) {
  bf16x8 cur[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) cur[d] = read_tr_operand(tile, kRowLd, 0, d * 32, lane);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    bf16x8 nxt[4];
    if (ks + 1 < KS) {
#pragma unroll
      for (int d = 0; d < 4; ++d) nxt[d] = read_tr_operand(tile, kRowLd, (ks + 1) * 16, d * 32, lane);
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) acc[d] = mfma32(cur[d], b[ks], acc[d]);
    ASPEC_STEP_FENCE();
    if (ks + 1 < KS) {
#pragma unroll
      for (int d = 0; d < 4; ++d) cur[d] = nxt[d];
    }
  }
}

__device__ __forceinline__ void store_row_c(uint16_t* dst, const f32x16 (&acc)[4], float mul, int g) {
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      u32x2 w;
      w.x = pack_bf16x2(acc[db][rq * 4 + 0] * mul, acc[db][rq * 4 + 1] * mul);
      w.y = pack_bf16x2(acc[db][rq * 4 + 2] * mul, acc[db][rq * 4 + 3] * mul);
      *reinterpret_cast<u32x2*>(dst + db * 32 + rq * 8 + g * 4) = w;
    }
  }
}

__device__ __forceinline__ void atomic_add_row_c(float* dst, const f32x16 (&acc)[4], int g) {
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) atomicAdd(dst + db * 32 + c_row(r, g), acc[db][r]);
  }
}

// ---------------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------------
template <bool PARTIAL>
__device__ __forceinline__ void fwd_tile(const uint16_t* sk, const uint16_t* sv,
                                         const bf16x8 (&qf)[8], f32x16 (&oacc)[4], float& m_run,
                                         float& l_run, const RowIntervals& iv, float scale_log2,
                                         int c, int g) {
  f32x16 s[2];
  mfma_chains2(s[0], s[1], sk + c * kRowLd + g * 8, sk + (32 + c) * kRowLd + g * 8, qf, qf,
               nullptr, nullptr);
  float tile_max = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = s[kb][r] * scale_log2;
      if (PARTIAL) x = iv.visible(kb * 32 + c_row(r, g)) ? x : -INFINITY;
      s[kb][r] = x;
      tile_max = fmaxf(tile_max, x);
    }
  }
  tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
  const bool grow = tile_max > m_run + kRescaleThreshold;
  if (__any(grow)) {
    const float m_new = grow ? tile_max : m_run;
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < 4; ++d) oacc[d] *= alpha;
  }
  float rowsum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(s[kb][r] - m_run);
      s[kb][r] = p;
      rowsum += p;
    }
  }
  l_run += rowsum;
  bf16x8 pb[4];
  pb[0] = pack_c_half(s[0], 0);
  pb[1] = pack_c_half(s[0], 8);
  pb[2] = pack_c_half(s[1], 0);
  pb[3] = pack_c_half(s[1], 8);
  mfma_tr_blocks<4>(oacc, sv, pb, g * 32 + c);
}

// One LDS buffer per workgroup (34 KB) with synchronous staging: two or more workgroups per CU
// hide each other's load latency, which pays more than register prefetch at this register budget.
template <int G>
__global__ void __launch_bounds__(kWave * G, 2) attn_fwd_kernel(AttnArgs a) {
  constexpr int NT = kWave * G;
  __shared__ __attribute__((aligned(16))) uint16_t s_k[kTN * kRowLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kTN * kRowLd];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t m = a.plan.nmf - 1 - blockIdx.x / a.hkv;  // longest prefixes first
  const int head = hkv * G + wave;
  const int64_t qrow = m * kTM + c;
  const bool valid_q = qrow < a.nq;
  const int64_t qsafe = valid_q ? qrow : a.nq - 1;

  bf16x8 qf[8];
  load_row_frag(qf, a.q + qsafe * a.qst + head * a.qsh, valid_q, g);
  int cb = a.ends[1 * a.nq + qsafe], ce = a.ends[2 * a.nq + qsafe];
  int db = a.ends[3 * a.nq + qsafe], de = a.ends[4 * a.nq + qsafe];
  if (!valid_q) cb = ce = db = de = 0;

  f32x16 oacc[4] = {};
  float m_run = kMaskValue;
  float l_run = 0.f;
  const uint16_t* kbase = a.k + hkv * a.ksh;
  const uint16_t* vbase = a.v + hkv * a.vsh;
  const int count = a.plan.f_cnt[m];
  const int32_t* list = a.plan.f_list + m * a.plan.nnf;

  for (int t = 0; t < count; ++t) {
    const uint32_t entry = static_cast<uint32_t>(list[t]);
    const int64_t key0 = static_cast<int64_t>(entry & ~kFullBit) * kTN;
    const int valid = static_cast<int>(min<int64_t>(kTN, a.nk - key0));
    __syncthreads();
    {
      TileLoader<NT, kTN> tile;
      tile.load(kbase + key0 * a.kst, a.kst, valid, tid);
      tile.store(s_k, nullptr, 0, tid);
      tile.load(vbase + key0 * a.vst, a.vst, valid, tid);
      tile.store(s_v, nullptr, 0, tid);
    }
    __syncthreads();
    if (entry & kFullBit) {
      RowIntervals iv{};
      fwd_tile<false>(s_k, s_v, qf, oacc, m_run, l_run, iv, a.scale_log2, c, g);
    } else {
      RowIntervals iv;
      iv.at_tile(static_cast<int>(key0), cb, ce, db, de);
      fwd_tile<true>(s_k, s_v, qf, oacc, m_run, l_run, iv, a.scale_log2, c, g);
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (valid_q) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    store_row_c(a.out + qrow * a.ost + head * a.osh, oacc, inv, g);
    if (g == 0) a.lse[static_cast<int64_t>(head) * a.nq + qrow] =
        l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : kMaskValue;
  }
}

// ---------------------------------------------------------------------------------------------
// Backward prepare: delta = rowsum(dO * O) - dLSE, lse2 = LSE * log2(e) (16 lanes per row).
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) attn_bwd_pre_kernel(AttnArgs a) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = t >> 4;  // row = head * nq + q
  const int chunk = static_cast<int>(t & 15);
  const bool valid = row < static_cast<int64_t>(a.hq) * a.nq;
  float acc = 0.f;
  if (valid) {
    const int64_t head = row / a.nq;
    const int64_t q = row - head * a.nq;
    const uint4 o = load16(a.o + q * a.ost + head * a.osh + chunk * 8);
    const uint4 d = load16(a.dout + q * a.dost + head * a.dosh + chunk * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += bf16_to_f32(half_of(o, e)) * bf16_to_f32(half_of(d, e));
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (valid && chunk == 0) {
    const float dl = a.dlse ? a.dlse[row] : 0.f;
    a.ws_delta[row] = acc - dl;
    a.ws_lse2[row] = a.lse_in[row] * kLog2e;
  }
}

// Grid: (key tile, kv head) pairs. Zeroes (ZERO) or converts to bf16 the fp32 accumulators of key
// tiles split over more than one unit; other tiles are written directly by their unit.
template <bool ZERO>
__global__ void __launch_bounds__(256) attn_bwd_acc_kernel(AttnArgs a) {
  const int hkv = blockIdx.x % a.hkv;
  const int64_t n = blockIdx.x / a.hkv;
  if (a.plan.b_chunks[n] <= 1) return;
  for (int i = threadIdx.x; i < kBwdTileN * (kHeadDim / 4); i += blockDim.x) {
    const int64_t key = n * kBwdTileN + i / (kHeadDim / 4);
    const int d = (i % (kHeadDim / 4)) * 4;
    if (key >= a.nk) continue;
    float* pk = a.ws_dk + (key * a.hkv + hkv) * kHeadDim + d;
    float* pv = a.ws_dv + (key * a.hkv + hkv) * kHeadDim + d;
    if (ZERO) {
      *reinterpret_cast<f32x4*>(pk) = f32x4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<f32x4*>(pv) = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(pk);
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(pv);
      u32x2 wk, wv;
      wk.x = pack_bf16x2(k4[0] * a.scale, k4[1] * a.scale);
      wk.y = pack_bf16x2(k4[2] * a.scale, k4[3] * a.scale);
      wv.x = pack_bf16x2(v4[0], v4[1]);
      wv.y = pack_bf16x2(v4[2], v4[3]);
      *reinterpret_cast<u32x2*>(a.dk + key * a.dkst + hkv * a.dksh + d) = wk;
      *reinterpret_cast<u32x2*>(a.dv + key * a.dvst + hkv * a.dvsh + d) = wv;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dQ: query-major, same traversal as the forward. dQ^T = K^T dS^T. One LDS buffer (so two
// workgroups share a CU) with the next tile prefetched into registers.
// ---------------------------------------------------------------------------------------------
template <bool PARTIAL>
__device__ __forceinline__ void dq_tile(const uint16_t* sk, const uint16_t* sv,
                                        const bf16x8 (&qf)[8], const bf16x8 (&df)[8],
                                        f32x16 (&dqacc)[4], float lse2, float delta,
                                        const RowIntervals& iv, float scale_log2, int c, int g) {
  bf16x8 dsb[4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    f32x16 s, dp;
    mfma_chains2(s, dp, sk + (kb * 32 + c) * kRowLd + g * 8, sv + (kb * 32 + c) * kRowLd + g * 8,
                 qf, df, nullptr, nullptr);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(s[r] * scale_log2 - lse2);
      if (PARTIAL) p = iv.visible(kb * 32 + c_row(r, g)) ? p : 0.f;
      s[r] = p * (dp[r] - delta);
    }
    dsb[kb * 2 + 0] = pack_c_half(s, 0);
    dsb[kb * 2 + 1] = pack_c_half(s, 8);
  }
  mfma_tr_blocks<4>(dqacc, sk, dsb, g * 32 + c);
}

template <int G>
__global__ void __launch_bounds__(kWave * G, 2) attn_bwd_dq_kernel(AttnArgs a) {
  constexpr int NT = kWave * G;
  __shared__ __attribute__((aligned(16))) uint16_t s_k[kTN * kRowLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kTN * kRowLd];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t m = a.plan.nmf - 1 - blockIdx.x / a.hkv;
  const int head = hkv * G + wave;
  const int64_t qrow = m * kTM + c;
  const bool valid_q = qrow < a.nq;
  const int64_t qsafe = valid_q ? qrow : a.nq - 1;

  bf16x8 qf[8], df[8];
  load_row_frag(qf, a.q + qsafe * a.qst + head * a.qsh, valid_q, g);
  load_row_frag(df, a.dout + qsafe * a.dost + head * a.dosh, valid_q, g);
  int cb = a.ends[1 * a.nq + qsafe], ce = a.ends[2 * a.nq + qsafe];
  int db = a.ends[3 * a.nq + qsafe], de = a.ends[4 * a.nq + qsafe];
  float lse2 = a.ws_lse2[static_cast<int64_t>(head) * a.nq + qsafe];
  float delta = a.ws_delta[static_cast<int64_t>(head) * a.nq + qsafe];
  if (!valid_q) {
    cb = ce = db = de = 0;
    lse2 = delta = 0.f;
  }

  f32x16 dqacc[4] = {};
  const uint16_t* kbase = a.k + hkv * a.ksh;
  const uint16_t* vbase = a.v + hkv * a.vsh;
  const int count = a.plan.f_cnt[m];
  const int32_t* list = a.plan.f_list + m * a.plan.nnf;

  for (int t = 0; t < count; ++t) {
    const uint32_t entry = static_cast<uint32_t>(list[t]);
    const int64_t key0 = static_cast<int64_t>(entry & ~kFullBit) * kTN;
    const int valid = static_cast<int>(min<int64_t>(kTN, a.nk - key0));
    __syncthreads();
    {
      TileLoader<NT, kTN> tile;
      tile.load(kbase + key0 * a.kst, a.kst, valid, tid);
      tile.store(s_k, nullptr, 0, tid);
      tile.load(vbase + key0 * a.vst, a.vst, valid, tid);
      tile.store(s_v, nullptr, 0, tid);
    }
    __syncthreads();
    if (entry & kFullBit) {
      RowIntervals iv{};
      dq_tile<false>(s_k, s_v, qf, df, dqacc, lse2, delta, iv, a.scale_log2, c, g);
    } else {
      RowIntervals iv;
      iv.at_tile(static_cast<int>(key0), cb, ce, db, de);
      dq_tile<true>(s_k, s_v, qf, df, dqacc, lse2, delta, iv, a.scale_log2, c, g);
    }
  }
  if (valid_q) store_row_c(a.dq + qrow * a.dqst + head * a.dqsh, dqacc, a.scale, g);
}

// ---------------------------------------------------------------------------------------------
// dK / dV: key-major. Each wave owns 32 keys of a 128-key tile. A work unit walks one chunk of the
// (descending) list of query tiles that see its key tile and, inside each query tile, all G heads
// of the KV group, so dK/dV are reduced over the GQA group in registers. A key tile covered by one
// unit is written directly; one split over several units is accumulated in fp32 and finalized.
// ---------------------------------------------------------------------------------------------
struct KvStage {
  uint16_t q[kBwdTileM * kRowLd];
  uint16_t dout[kBwdTileM * kRowLd];
  float lse2[kBwdTileM];
  float delta[kBwdTileM];
  int4 ends[kBwdTileM];
};

// krow / vrow: this lane's key row of the LDS-resident K and V tiles, at dim offset g*8.
template <bool PARTIAL>
__device__ __forceinline__ void dkdv_iter(const KvStage& s, const uint16_t* krow,
                                          const uint16_t* vrow, f32x16 (&dkacc)[4],
                                          f32x16 (&dvacc)[4], int ikey, float scale_log2, int c,
                                          int g) {
  // S = Q K^T and dP = dO V^T; C layout: lane <-> this wave's key, rows <-> queries.
  f32x16 sacc, dp;
  mfma_chains2(sacc, dp, s.q + c * kRowLd + g * 8, s.dout + c * kRowLd + g * 8, nullptr, nullptr,
               krow, vrow);
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
    const int r0 = rq * 8 + g * 4;
    const f32x4 l4 = *reinterpret_cast<const f32x4*>(s.lse2 + r0);
    const f32x4 d4 = *reinterpret_cast<const f32x4*>(s.delta + r0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = rq * 4 + j;
      float p = fast_exp2(sacc[r] * scale_log2 - l4[j]);
      if (PARTIAL) {
        const int4 e = s.ends[r0 + j];
        p = interval_visible(ikey, e.x, e.y, e.z, e.w) ? p : 0.f;
      }
      sacc[r] = p;
      dp[r] = p * (dp[r] - d4[j]);
    }
  }
  const bf16x8 pp[2] = {pack_c_half(sacc, 0), pack_c_half(sacc, 8)};
  const bf16x8 dd[2] = {pack_c_half(dp, 0), pack_c_half(dp, 8)};
  mfma_tr_blocks<2>(dvacc, s.dout, pp, g * 32 + c);
  mfma_tr_blocks<2>(dkacc, s.q, dd, g * 32 + c);
}

__global__ void __launch_bounds__(kWave * kKvWaves) attn_bwd_dkdv_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) KvStage st[2];
  __shared__ __attribute__((aligned(16))) uint16_t s_key[kBwdTileN * kRowLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_val[kBwdTileN * kRowLd];
  // An AGPR operand anywhere in the kernel makes instruction selection emit the AGPR form of the
  // MFMAs, so the dK/dV accumulators stay in AGPRs across the walk instead of being copied in
  // and out of VGPRs every iteration.
  asm volatile("" ::"a"(0));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t u = blockIdx.x / a.hkv;
  if (u >= a.plan.b_nunits[0]) return;
  const int32_t unit = a.plan.b_units[u];
  const int64_t n = unit >> kUnitChunkBits;
  const int chunk = unit & ((1 << kUnitChunkBits) - 1);
  const int count = a.plan.b_cnt[n];
  const int first = chunk * kBwdChunk;
  const int last = min(count, first + kBwdChunk);
  const int iters = max(0, last - first) * a.group;
  const int32_t* list = a.plan.b_list + n * a.plan.nmb;

  const int64_t key = n * kBwdTileN + wave * 32 + c;
  const bool valid_k = key < a.nk;
  {
    // The unit's 128 keys of K and V stay in LDS for the whole walk (keys past K are zero).
    const int64_t key0 = n * kBwdTileN;
    const int valid = static_cast<int>(min<int64_t>(kBwdTileN, a.nk - key0));
    TileLoader<kWave * kKvWaves, kBwdTileN> tile;
    tile.load(a.k + key0 * a.kst + hkv * a.ksh, a.kst, valid, tid);
    tile.store(s_key, nullptr, 0, tid);
    tile.load(a.v + key0 * a.vst + hkv * a.vsh, a.vst, valid, tid);
    tile.store(s_val, nullptr, 0, tid);
  }
  const uint16_t* krow = s_key + (wave * 32 + c) * kRowLd + g * 8;
  const uint16_t* vrow = s_val + (wave * 32 + c) * kRowLd + g * 8;
  f32x16 dkacc[4] = {};
  f32x16 dvacc[4] = {};
  const int ikey = static_cast<int>(key);

  // Staging roles: threads [0,128) Q rows, [128,256) dO rows, [0,32) also the row scalars.
  TileLoader<128, kBwdTileM> rows;
  float sc_lse2 = 0.f, sc_delta = 0.f;
  int4 sc_ends = make_int4(0, 0, 0, 0);
  const bool loads_q = tid < 128;
  const int rtid = loads_q ? tid : tid - 128;
  auto fetch = [&](int i) {
    const int64_t q0 = static_cast<int64_t>(list[first + i / a.group] & ~kFullBit) * kBwdTileM;
    const int head = hkv * a.group + i % a.group;
    const int valid = static_cast<int>(min<int64_t>(kBwdTileM, a.nq - q0));
    if (loads_q) rows.load(a.q + q0 * a.qst + head * a.qsh, a.qst, valid, rtid);
    else rows.load(a.dout + q0 * a.dost + head * a.dosh, a.dost, valid, rtid);
    if (tid < kBwdTileM) {
      const bool ok = tid < valid;
      const int64_t qr = q0 + (ok ? tid : valid - 1);
      const int64_t idx = static_cast<int64_t>(head) * a.nq + qr;
      sc_lse2 = ok ? a.ws_lse2[idx] : 0.f;
      sc_delta = ok ? a.ws_delta[idx] : 0.f;
      const int4 e = make_int4(a.ends[1 * a.nq + qr], a.ends[2 * a.nq + qr], a.ends[3 * a.nq + qr],
                               a.ends[4 * a.nq + qr]);
      sc_ends = ok ? e : make_int4(0, 0, 0, 0);
    }
  };
  auto put = [&](KvStage& s) {
    if (loads_q) rows.store(s.q, nullptr, 0, rtid);
    else rows.store(s.dout, nullptr, 0, rtid);
    if (tid < kBwdTileM) {
      s.lse2[tid] = sc_lse2;
      s.delta[tid] = sc_delta;
      s.ends[tid] = sc_ends;
    }
  };
  if (iters > 0) {
    fetch(0);
    put(st[0]);
    if (iters > 1) fetch(1);
  }
  __syncthreads();

  for (int i = 0; i < iters; ++i) {
    const KvStage& s = st[i & 1];
    // One masked code path: the per-row interval test is cheap next to this iteration's 32 MFMAs,
    // and a single body keeps the accumulators' register assignment stable across the loop.
    dkdv_iter<true>(s, krow, vrow, dkacc, dvacc, ikey, a.scale_log2, c, g);
    if (i + 1 < iters) put(st[(i + 1) & 1]);
    if (i + 2 < iters) fetch(i + 2);
    __syncthreads();
  }
  if (!valid_k) return;
  if (a.plan.b_chunks[n] == 1) {
    store_row_c(a.dk + key * a.dkst + hkv * a.dksh, dkacc, a.scale, g);
    store_row_c(a.dv + key * a.dvst + hkv * a.dvsh, dvacc, 1.f, g);
  } else {
    atomic_add_row_c(a.ws_dk + (key * a.hkv + hkv) * kHeadDim, dkacc, g);
    atomic_add_row_c(a.ws_dv + (key * a.hkv + hkv) * kHeadDim, dvacc, g);
  }
}

int validate(const AttnArgs& a, int64_t head_dim) {
  if (head_dim != kHeadDim)
    return set_error(ASPEC_ERR_UNSUPPORTED, "DSpark attention supports head_dim 128 only, got %lld",
                     (long long)head_dim);
  if (a.nq <= 0 || a.nk <= 0 || a.hq <= 0 || a.hkv <= 0)
    return set_error(ASPEC_ERR_INVALID, "DSpark attention needs positive sizes");
  if (a.hq % a.hkv)
    return set_error(ASPEC_ERR_INVALID, "query heads must be divisible by the matching KV head count");
  if (a.group > kMaxGroup)
    return set_error(ASPEC_ERR_UNSUPPORTED, "GQA group %d exceeds %d", a.group, kMaxGroup);
  if (a.nk >= (1LL << 31) - kBwdTileN)
    return set_error(ASPEC_ERR_INVALID, "too many keys for int32 tile indexing");
  return ASPEC_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool stride_ok(int64_t s) { return s % 8 == 0; }

#define ASPEC_GROUP_DISPATCH(KERNEL, GROUP, GRID, STREAM, ARGS)                                  \
  switch (GROUP) {                                                                              \
    case 1: hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(kWave * 1), 0, STREAM, ARGS); break;       \
    case 2: hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(kWave * 2), 0, STREAM, ARGS); break;       \
    case 3: hipLaunchKernelGGL(KERNEL<3>, GRID, dim3(kWave * 3), 0, STREAM, ARGS); break;       \
    case 4: hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(kWave * 4), 0, STREAM, ARGS); break;       \
    case 5: hipLaunchKernelGGL(KERNEL<5>, GRID, dim3(kWave * 5), 0, STREAM, ARGS); break;       \
    case 6: hipLaunchKernelGGL(KERNEL<6>, GRID, dim3(kWave * 6), 0, STREAM, ARGS); break;       \
    case 7: hipLaunchKernelGGL(KERNEL<7>, GRID, dim3(kWave * 7), 0, STREAM, ARGS); break;       \
    default: hipLaunchKernelGGL(KERNEL<8>, GRID, dim3(kWave * 8), 0, STREAM, ARGS); break;      \
  }

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_dspark_attn_fwd(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                                     const void* k, int64_t k_stride_token, int64_t k_stride_head,
                                     const void* v, int64_t v_stride_token, int64_t v_stride_head,
                                     const int32_t* endpoints, const void* plan,
                                     int64_t num_queries, int64_t num_keys, int64_t q_heads,
                                     int64_t kv_heads, int64_t head_dim, float scale, void* out,
                                     int64_t o_stride_token, int64_t o_stride_head, float* lse,
                                     void* stream) {
  AttnArgs a = {};
  a.q = static_cast<const uint16_t*>(q); a.qst = q_stride_token; a.qsh = q_stride_head;
  a.k = static_cast<const uint16_t*>(k); a.kst = k_stride_token; a.ksh = k_stride_head;
  a.v = static_cast<const uint16_t*>(v); a.vst = v_stride_token; a.vsh = v_stride_head;
  a.ends = endpoints;
  a.nq = num_queries; a.nk = num_keys;
  a.hq = static_cast<int>(q_heads); a.hkv = static_cast<int>(kv_heads);
  a.group = kv_heads > 0 ? static_cast<int>(q_heads / kv_heads) : 0;
  a.scale = scale; a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t*>(out); a.ost = o_stride_token; a.osh = o_stride_head;
  a.lse = lse;
  int rc = validate(a, head_dim);
  if (rc) return rc;
  if (!q || !k || !v || !out || !lse || !endpoints || !plan)
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to DSpark attention forward");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) ||
      !stride_ok(q_stride_token) || !stride_ok(q_stride_head) || !stride_ok(k_stride_token) ||
      !stride_ok(k_stride_head) || !stride_ok(v_stride_token) || !stride_ok(v_stride_head) ||
      !stride_ok(o_stride_token) || !stride_ok(o_stride_head))
    return set_error(ASPEC_ERR_INVALID, "DSpark attention needs 16-byte aligned rows");
  a.plan = plan_view(const_cast<void*>(plan), num_queries, num_keys);
  const dim3 grid(static_cast<uint32_t>(a.plan.nmf * a.hkv));
  hipStream_t s = static_cast<hipStream_t>(stream);
  ASPEC_GROUP_DISPATCH(attn_fwd_kernel, a.group, grid, s, a);
  return check_launch("attn_fwd_kernel");
}

extern "C" int aspec_dspark_attn_bwd_workspace_bytes(int64_t num_queries, int64_t num_keys,
                                                     int64_t q_heads, int64_t kv_heads,
                                                     size_t* bytes) {
  if (num_queries <= 0 || num_keys <= 0 || q_heads <= 0 || kv_heads <= 0 || !bytes)
    return set_error(ASPEC_ERR_INVALID, "workspace size needs positive sizes");
  *bytes = static_cast<size_t>(2 * num_queries * q_heads + 2 * num_keys * kv_heads * kHeadDim) *
           sizeof(float);
  return ASPEC_OK;
}

extern "C" int aspec_dspark_attn_bwd_stages(
    int stages, const void* q, int64_t q_stride_token, int64_t q_stride_head, const void* k,
    int64_t k_stride_token, int64_t k_stride_head, const void* v, int64_t v_stride_token,
    int64_t v_stride_head, const void* out, int64_t o_stride_token, int64_t o_stride_head,
    const void* dout, int64_t do_stride_token, int64_t do_stride_head, const float* lse,
    const float* dlse, const int32_t* endpoints, const void* plan, int64_t num_queries,
    int64_t num_keys, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float scale, void* dq,
    int64_t dq_stride_token, int64_t dq_stride_head, void* dk, int64_t dk_stride_token,
    int64_t dk_stride_head, void* dv, int64_t dv_stride_token, int64_t dv_stride_head,
    void* workspace, void* stream) {
  if (stages <= 0 || stages > 15) return set_error(ASPEC_ERR_INVALID, "backward stage mask must be 1..15");
  AttnArgs a = {};
  a.q = static_cast<const uint16_t*>(q); a.qst = q_stride_token; a.qsh = q_stride_head;
  a.k = static_cast<const uint16_t*>(k); a.kst = k_stride_token; a.ksh = k_stride_head;
  a.v = static_cast<const uint16_t*>(v); a.vst = v_stride_token; a.vsh = v_stride_head;
  a.o = static_cast<const uint16_t*>(out); a.ost = o_stride_token; a.osh = o_stride_head;
  a.dout = static_cast<const uint16_t*>(dout); a.dost = do_stride_token; a.dosh = do_stride_head;
  a.ends = endpoints;
  a.nq = num_queries; a.nk = num_keys;
  a.hq = static_cast<int>(q_heads); a.hkv = static_cast<int>(kv_heads);
  a.group = kv_heads > 0 ? static_cast<int>(q_heads / kv_heads) : 0;
  a.scale = scale; a.scale_log2 = scale * kLog2e;
  a.lse_in = lse; a.dlse = dlse;
  a.dq = static_cast<uint16_t*>(dq); a.dqst = dq_stride_token; a.dqsh = dq_stride_head;
  a.dk = static_cast<uint16_t*>(dk); a.dkst = dk_stride_token; a.dksh = dk_stride_head;
  a.dv = static_cast<uint16_t*>(dv); a.dvst = dv_stride_token; a.dvsh = dv_stride_head;
  int rc = validate(a, head_dim);
  if (rc) return rc;
  if (!q || !k || !v || !out || !dout || !lse || !endpoints || !plan || !dq || !dk || !dv || !workspace)
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to DSpark attention backward");
  const void* ptrs[] = {q, k, v, out, dout, dq, dk, dv, workspace};
  for (const void* p : ptrs)
    if (!aligned16(p)) return set_error(ASPEC_ERR_INVALID, "DSpark attention needs 16-byte aligned rows");
  const int64_t strides[] = {q_stride_token, q_stride_head, k_stride_token, k_stride_head,
                             v_stride_token, v_stride_head, o_stride_token, o_stride_head,
                             do_stride_token, do_stride_head, dq_stride_token, dq_stride_head,
                             dk_stride_token, dk_stride_head, dv_stride_token, dv_stride_head};
  for (int64_t s : strides)
    if (!stride_ok(s)) return set_error(ASPEC_ERR_INVALID, "DSpark attention needs 16-byte aligned rows");
  a.ws_delta = static_cast<float*>(workspace);
  a.ws_lse2 = a.ws_delta + num_queries * q_heads;
  a.ws_dk = a.ws_lse2 + num_queries * q_heads;
  a.ws_dv = a.ws_dk + num_keys * kv_heads * kHeadDim;
  a.plan = plan_view(const_cast<void*>(plan), num_queries, num_keys);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 acc_grid(static_cast<uint32_t>(a.plan.nnb * a.hkv));

  if (stages & 1) {
    const int64_t pre_threads = num_queries * q_heads * 16;
    hipLaunchKernelGGL(attn_bwd_pre_kernel, dim3(static_cast<uint32_t>((pre_threads + 255) / 256)),
                       dim3(256), 0, s, a);
    if ((rc = check_launch("attn_bwd_pre_kernel"))) return rc;
    hipLaunchKernelGGL(attn_bwd_acc_kernel<true>, acc_grid, dim3(256), 0, s, a);
    if ((rc = check_launch("attn_bwd_acc_kernel<zero>"))) return rc;
  }
  if (stages & 2) {
    const dim3 grid(static_cast<uint32_t>(a.plan.nmf * a.hkv));
    ASPEC_GROUP_DISPATCH(attn_bwd_dq_kernel, a.group, grid, s, a);
    if ((rc = check_launch("attn_bwd_dq_kernel"))) return rc;
  }
  if (stages & 4) {
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel, dim3(static_cast<uint32_t>(a.plan.max_units * a.hkv)),
                       dim3(kWave * kKvWaves), 0, s, a);
    if ((rc = check_launch("attn_bwd_dkdv_kernel"))) return rc;
  }
  if (stages & 8) {
    hipLaunchKernelGGL(attn_bwd_acc_kernel<false>, acc_grid, dim3(256), 0, s, a);
    rc = check_launch("attn_bwd_acc_kernel<finalize>");
  }
  return rc;
}

extern "C" int aspec_dspark_attn_bwd(
    const void* q, int64_t q_stride_token, int64_t q_stride_head, const void* k,
    int64_t k_stride_token, int64_t k_stride_head, const void* v, int64_t v_stride_token,
    int64_t v_stride_head, const void* out, int64_t o_stride_token, int64_t o_stride_head,
    const void* dout, int64_t do_stride_token, int64_t do_stride_head, const float* lse,
    const float* dlse, const int32_t* endpoints, const void* plan, int64_t num_queries,
    int64_t num_keys, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float scale, void* dq,
    int64_t dq_stride_token, int64_t dq_stride_head, void* dk, int64_t dk_stride_token,
    int64_t dk_stride_head, void* dv, int64_t dv_stride_token, int64_t dv_stride_head,
    void* workspace, void* stream) {
  return aspec_dspark_attn_bwd_stages(
      15, q, q_stride_token, q_stride_head, k, k_stride_token, k_stride_head, v, v_stride_token,
      v_stride_head, out, o_stride_token, o_stride_head, dout, do_stride_token, do_stride_head,
      lse, dlse, endpoints, plan, num_queries, num_keys, q_heads, kv_heads, head_dim, scale, dq,
      dq_stride_token, dq_stride_head, dk, dk_stride_token, dk_stride_head, dv, dv_stride_token,
      dv_stride_head, workspace, stream);
}
