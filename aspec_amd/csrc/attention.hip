// DSpark block-sparse attention on gfx950: forward, backward preprocess, dQ and dK/dV kernels.
//
// Masking semantics (direct_cp.py:382-425 / thd_attention.py:77-131, as interval endpoints from
// direct_cp.py:750-900): query row q sees key k iff cb[q] <= k < ce[q] or db[q] <= k < de[q].
// Only tiles listed in the plan are visited; "full" tiles skip the predicate.
//
// One workgroup stacks the G = Hq/Hkv query heads of one KV head (one wave per head) so each K/V
// tile is staged in LDS once for the whole GQA group. Scores are computed transposed
// (S^T = K Q^T) so each lane owns one query row: the softmax statistics are per-lane scalars and
// P^T feeds the P.V MFMA straight from registers.
#include "attn_common.h"
#include "plan.h"

namespace aspec {
namespace {

constexpr int kTM = kFwdTileM;          // query rows per wave (one per lane column)
constexpr int kTN = kFwdTileN;          // keys per tile
constexpr int kVtLd = kTN + 4;          // transposed 64-key tile stride (136 B)
constexpr int kQtLd = kBwdTileM + 4;    // transposed 32-row tile stride (72 B)
constexpr int kMaxGroup = 8;

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
  uint16_t* dq; int64_t dqst, dqsh;
  uint16_t* dk; int64_t dkst, dksh;
  uint16_t* dv; int64_t dvst, dvsh;
};

__device__ __forceinline__ void load_row_frag(bf16x8 (&frag)[8], const uint16_t* base, bool valid,
                                              int g) {
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) {
    frag[ds] = valid ? as_bf16x8(load16(base + ds * 16 + g * 8)) : as_bf16x8(make_uint4(0, 0, 0, 0));
  }
}

// S^T block (32 keys x 32 queries) = K_tile[kb*32 .. +32] . Q^T, K row-major in LDS.
__device__ __forceinline__ f32x16 scores_t(const uint16_t* tile, int kb, const bf16x8 (&qf)[8],
                                           int c, int g) {
  f32x16 acc = {};
  const uint16_t* row = tile + (kb * 32 + c) * kRowLd + g * 8;
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) acc = mfma32(as_bf16x8(load16(row + ds * 16)), qf[ds], acc);
  return acc;
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

// ---------------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kWave * kMaxGroup) attn_fwd_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t s_k[kTN * kRowLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_vt[kHeadDim * kVtLd];

  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t m = a.plan.nmf - 1 - blockIdx.x / a.hkv;  // longest prefixes first
  const int head = hkv * a.group + wave;
  const int64_t qrow = m * kTM + c;
  const bool valid_q = qrow < a.nq;

  bf16x8 qf[8];
  load_row_frag(qf, a.q + qrow * a.qst + head * a.qsh, valid_q, g);
  int cb = 0, ce = 0, db = 0, de = 0;
  if (valid_q) {
    cb = a.ends[1 * a.nq + qrow];
    ce = a.ends[2 * a.nq + qrow];
    db = a.ends[3 * a.nq + qrow];
    de = a.ends[4 * a.nq + qrow];
  }

  f32x16 oacc[4] = {};
  float m_run = kMaskValue;
  float l_run = 0.f;
  const uint16_t* kbase = a.k + hkv * a.ksh;
  const uint16_t* vbase = a.v + hkv * a.vsh;

  for (int pass = 0; pass < 2; ++pass) {
    const bool partial = pass == 1;
    const int count = partial ? a.plan.f_pcnt[m] : a.plan.f_fcnt[m];
    const int32_t* list = (partial ? a.plan.f_pidx : a.plan.f_fidx) + m * a.plan.nnf;
    for (int t = 0; t < count; ++t) {
      const int64_t key0 = static_cast<int64_t>(list[t]) * kTN;
      __syncthreads();
      stage_tile(kbase, a.kst, key0, a.nk, kTN, s_k, nullptr, 0, tid, nthreads);
      stage_tile(vbase, a.vst, key0, a.nk, kTN, nullptr, s_vt, kVtLd, tid, nthreads);
      __syncthreads();

      f32x16 s[2];
      s[0] = scores_t(s_k, 0, qf, c, g);
      s[1] = scores_t(s_k, 1, qf, c, g);
      float tile_max = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[kb][r] * a.scale_log2;
          if (partial) {
            const int key = static_cast<int>(key0) + kb * 32 + c_row(r, g);
            x = interval_visible(key, cb, ce, db, de) ? x : -INFINITY;
          }
          s[kb][r] = x;
          tile_max = fmaxf(tile_max, x);
        }
      }
      tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
      const float m_new = fmaxf(m_run, tile_max);
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      float rowsum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = exp2f(s[kb][r] - m_new);
          s[kb][r] = p;
          rowsum += p;
        }
      }
      l_run = l_run * alpha + rowsum;
#pragma unroll
      for (int d = 0; d < 4; ++d) oacc[d] *= alpha;

      bf16x8 pb[4];
      pb[0] = pack_c_half(s[0], 0);
      pb[1] = pack_c_half(s[0], 8);
      pb[2] = pack_c_half(s[1], 0);
      pb[3] = pack_c_half(s[1], 8);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint16_t* vrow = s_vt + (d * 32 + c) * kVtLd;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) oacc[d] = mfma32(read_split_operand(vrow + ks * 16, g), pb[ks], oacc[d]);
      }
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
// Backward preprocess: delta = rowsum(dO * O) - dLSE, lse2 = LSE * log2(e). 16 lanes per row.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) attn_bwd_pre_kernel(AttnArgs a) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = t >> 4;  // row = head * nq + q
  const int chunk = static_cast<int>(t & 15);
  const bool valid = row < static_cast<int64_t>(a.hq) * a.nq;
  float acc = 0.f;
  int64_t head = 0, q = 0;
  if (valid) {
    head = row / a.nq;
    q = row - head * a.nq;
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

// ---------------------------------------------------------------------------------------------
// dQ: query-major, same traversal as the forward. dQ^T = K^T dS^T.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kWave * kMaxGroup) attn_bwd_dq_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t s_k[kTN * kRowLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_kt[kHeadDim * kVtLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kTN * kRowLd];

  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t m = a.plan.nmf - 1 - blockIdx.x / a.hkv;
  const int head = hkv * a.group + wave;
  const int64_t qrow = m * kTM + c;
  const bool valid_q = qrow < a.nq;

  bf16x8 qf[8], df[8];
  load_row_frag(qf, a.q + qrow * a.qst + head * a.qsh, valid_q, g);
  load_row_frag(df, a.dout + qrow * a.dost + head * a.dosh, valid_q, g);
  int cb = 0, ce = 0, db = 0, de = 0;
  float lse2 = 0.f, delta = 0.f;
  if (valid_q) {
    cb = a.ends[1 * a.nq + qrow];
    ce = a.ends[2 * a.nq + qrow];
    db = a.ends[3 * a.nq + qrow];
    de = a.ends[4 * a.nq + qrow];
    lse2 = a.ws_lse2[static_cast<int64_t>(head) * a.nq + qrow];
    delta = a.ws_delta[static_cast<int64_t>(head) * a.nq + qrow];
  }

  f32x16 dqacc[4] = {};
  const uint16_t* kbase = a.k + hkv * a.ksh;
  const uint16_t* vbase = a.v + hkv * a.vsh;
  for (int pass = 0; pass < 2; ++pass) {
    const bool partial = pass == 1;
    const int count = partial ? a.plan.f_pcnt[m] : a.plan.f_fcnt[m];
    const int32_t* list = (partial ? a.plan.f_pidx : a.plan.f_fidx) + m * a.plan.nnf;
    for (int t = 0; t < count; ++t) {
      const int64_t key0 = static_cast<int64_t>(list[t]) * kTN;
      __syncthreads();
      stage_tile(kbase, a.kst, key0, a.nk, kTN, s_k, s_kt, kVtLd, tid, nthreads);
      stage_tile(vbase, a.vst, key0, a.nk, kTN, s_v, nullptr, 0, tid, nthreads);
      __syncthreads();

      bf16x8 dsb[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x16 s = scores_t(s_k, kb, qf, c, g);
        f32x16 dp = scores_t(s_v, kb, df, c, g);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = exp2f(s[r] * a.scale_log2 - lse2);
          if (partial) {
            const int key = static_cast<int>(key0) + kb * 32 + c_row(r, g);
            p = interval_visible(key, cb, ce, db, de) ? p : 0.f;
          }
          s[r] = p * (dp[r] - delta);
        }
        dsb[kb * 2 + 0] = pack_c_half(s, 0);
        dsb[kb * 2 + 1] = pack_c_half(s, 8);
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint16_t* krow = s_kt + (d * 32 + c) * kVtLd;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) dqacc[d] = mfma32(read_split_operand(krow + ks * 16, g), dsb[ks], dqacc[d]);
      }
    }
  }
  if (valid_q) store_row_c(a.dq + qrow * a.dqst + head * a.dqsh, dqacc, a.scale, g);
}

// ---------------------------------------------------------------------------------------------
// dK / dV: key-major. Each wave owns 32 keys; the workgroup walks the query tiles that see its
// 128-key tile and, inside each, all G heads of the KV group, so dK/dV are reduced over the
// GQA group in registers and written once.
// ---------------------------------------------------------------------------------------------
constexpr int kKvWaves = kBwdTileN / 32;

__global__ void __launch_bounds__(kWave * kKvWaves) attn_bwd_dkdv_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t s_q[kBwdTileM * kRowLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_qt[kHeadDim * kQtLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_do[kBwdTileM * kRowLd];
  __shared__ __attribute__((aligned(16))) uint16_t s_dot[kHeadDim * kQtLd];
  __shared__ __attribute__((aligned(16))) float s_lse2[kBwdTileM];
  __shared__ __attribute__((aligned(16))) float s_delta[kBwdTileM];
  __shared__ __attribute__((aligned(16))) int32_t s_ends[4][kBwdTileM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t n = blockIdx.x / a.hkv;
  const int64_t key = n * kBwdTileN + wave * 32 + c;
  const bool valid_k = key < a.nk;

  bf16x8 kf[8], vf[8];
  load_row_frag(kf, a.k + key * a.kst + hkv * a.ksh, valid_k, g);
  load_row_frag(vf, a.v + key * a.vst + hkv * a.vsh, valid_k, g);
  f32x16 dkacc[4] = {};
  f32x16 dvacc[4] = {};
  const int ikey = static_cast<int>(key);

  for (int pass = 0; pass < 2; ++pass) {
    const bool partial = pass == 1;
    const int count = partial ? a.plan.b_pcnt[n] : a.plan.b_fcnt[n];
    const int32_t* list = (partial ? a.plan.b_pidx : a.plan.b_fidx) + n * a.plan.nmb;
    for (int t = 0; t < count; ++t) {
      const int64_t q0 = static_cast<int64_t>(list[t]) * kBwdTileM;
      for (int j = 0; j < a.group; ++j) {
        const int head = hkv * a.group + j;
        __syncthreads();
        // threads [0,128) stage Q, [128,256) stage dO
        if (tid < 128) {
          stage_tile(a.q + head * a.qsh, a.qst, q0, a.nq, kBwdTileM, s_q, s_qt, kQtLd, tid, 128);
        } else {
          stage_tile(a.dout + head * a.dosh, a.dost, q0, a.nq, kBwdTileM, s_do, s_dot, kQtLd, tid - 128, 128);
        }
        if (tid < kBwdTileM) {
          const int64_t qr = q0 + tid;
          const bool ok = qr < a.nq;
          const int64_t idx = static_cast<int64_t>(head) * a.nq + qr;
          s_lse2[tid] = ok ? a.ws_lse2[idx] : 0.f;
          s_delta[tid] = ok ? a.ws_delta[idx] : 0.f;
          s_ends[0][tid] = ok ? a.ends[1 * a.nq + qr] : 0;
          s_ends[1][tid] = ok ? a.ends[2 * a.nq + qr] : 0;
          s_ends[2][tid] = ok ? a.ends[3 * a.nq + qr] : 0;
          s_ends[3][tid] = ok ? a.ends[4 * a.nq + qr] : 0;
        }
        __syncthreads();

        // S = Q K^T and dP = dO V^T; C layout: lane <-> this wave's key, rows <-> queries.
        f32x16 s = {}, dp = {};
        const uint16_t* qrow = s_q + c * kRowLd + g * 8;
        const uint16_t* drow = s_do + c * kRowLd + g * 8;
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) {
          s = mfma32(as_bf16x8(load16(qrow + ds * 16)), kf[ds], s);
          dp = mfma32(as_bf16x8(load16(drow + ds * 16)), vf[ds], dp);
        }
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int r0 = rq * 8 + g * 4;
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(s_lse2 + r0);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(s_delta + r0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = rq * 4 + i;
            float p = exp2f(s[r] * a.scale_log2 - l4[i]);
            if (partial) {
              const int qq = r0 + i;
              p = interval_visible(ikey, s_ends[0][qq], s_ends[1][qq], s_ends[2][qq], s_ends[3][qq]) ? p : 0.f;
            }
            s[r] = p;
            dp[r] = p * (dp[r] - d4[i]);
          }
        }
        const bf16x8 p0 = pack_c_half(s, 0), p1 = pack_c_half(s, 8);
        const bf16x8 d0 = pack_c_half(dp, 0), d1 = pack_c_half(dp, 8);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint16_t* dot = s_dot + (d * 32 + c) * kQtLd;
          const uint16_t* qt = s_qt + (d * 32 + c) * kQtLd;
          dvacc[d] = mfma32(read_split_operand(dot, g), p0, dvacc[d]);
          dvacc[d] = mfma32(read_split_operand(dot + 16, g), p1, dvacc[d]);
          dkacc[d] = mfma32(read_split_operand(qt, g), d0, dkacc[d]);
          dkacc[d] = mfma32(read_split_operand(qt + 16, g), d1, dkacc[d]);
        }
      }
    }
  }
  if (valid_k) {
    store_row_c(a.dk + key * a.dkst + hkv * a.dksh, dkacc, a.scale, g);
    store_row_c(a.dv + key * a.dvst + hkv * a.dvsh, dvacc, 1.f, g);
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

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_dspark_plan_bytes(int64_t num_queries, int64_t num_keys, size_t* bytes) {
  if (num_queries <= 0 || num_keys <= 0 || !bytes)
    return set_error(ASPEC_ERR_INVALID, "plan size needs positive query/key counts");
  *bytes = plan_view(nullptr, num_queries, num_keys).bytes;
  return ASPEC_OK;
}

extern "C" int aspec_dspark_plan_build(const int32_t* endpoints, int64_t num_queries,
                                       int64_t num_keys, void* plan, void* stream) {
  if (num_queries <= 0 || num_keys <= 0 || !endpoints || !plan)
    return set_error(ASPEC_ERR_INVALID, "plan build needs endpoints, a plan buffer and sizes");
  const PlanView p = plan_view(plan, num_queries, num_keys);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = launch_tile_metadata(endpoints, num_queries, num_keys, kFwdTileM, kFwdTileN, 0,
                                p.f_classes, p.f_pcnt, p.f_pidx, p.f_fcnt, p.f_fidx, nullptr,
                                nullptr, nullptr, nullptr, s);
  if (rc) return rc;
  return launch_tile_metadata(endpoints, num_queries, num_keys, kBwdTileM, kBwdTileN, 0,
                              p.b_classes, nullptr, nullptr, nullptr, nullptr, p.b_pcnt, p.b_pidx,
                              p.b_fcnt, p.b_fidx, s);
}

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
  const int64_t blocks = a.plan.nmf * a.hkv;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kWave * a.group), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("attn_fwd_kernel");
}

extern "C" int aspec_dspark_attn_bwd_workspace_bytes(int64_t num_queries, int64_t q_heads,
                                                     size_t* bytes) {
  if (num_queries <= 0 || q_heads <= 0 || !bytes)
    return set_error(ASPEC_ERR_INVALID, "workspace size needs positive sizes");
  *bytes = static_cast<size_t>(2 * num_queries * q_heads) * sizeof(float);
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
  if (stages <= 0 || stages > 7) return set_error(ASPEC_ERR_INVALID, "backward stage mask must be 1..7");
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
  const void* ptrs[] = {q, k, v, out, dout, dq, dk, dv};
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
  a.plan = plan_view(const_cast<void*>(plan), num_queries, num_keys);
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (stages & 1) {
    const int64_t pre_threads = num_queries * q_heads * 16;
    hipLaunchKernelGGL(attn_bwd_pre_kernel, dim3(static_cast<uint32_t>((pre_threads + 255) / 256)),
                       dim3(256), 0, s, a);
    rc = check_launch("attn_bwd_pre_kernel");
    if (rc) return rc;
  }
  if (stages & 2) {
    hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3(static_cast<uint32_t>(a.plan.nmf * a.hkv)),
                       dim3(kWave * a.group), 0, s, a);
    rc = check_launch("attn_bwd_dq_kernel");
    if (rc) return rc;
  }
  if (stages & 4) {
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel, dim3(static_cast<uint32_t>(a.plan.nnb * a.hkv)),
                       dim3(kWave * kKvWaves), 0, s, a);
    rc = check_launch("attn_bwd_dkdv_kernel");
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
      7, q, q_stride_token, q_stride_head, k, k_stride_token, k_stride_head, v, v_stride_token,
      v_stride_head, out, o_stride_token, o_stride_head, dout, do_stride_token, do_stride_head,
      lse, dlse, endpoints, plan, num_queries, num_keys, q_heads, kv_heads, head_dim, scale, dq,
      dq_stride_token, dq_stride_head, dk, dk_stride_token, dk_stride_head, dv, dv_stride_token,
      dv_stride_head, workspace, stream);
}
