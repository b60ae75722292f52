// Vocabulary-sliced loss kernels: softmax-L1 (tiled_l1.py semantics) and cross-entropy, forward
// and backward, alone or fused. HBM-bound streaming reductions.
//
// Forward:
//   row walk (V % 8 == 0, V <= 512*8*8): one 512-thread workgroup per CU walks the rows; each row
//   of draft and teacher logits is read from HBM exactly once into registers while the previous
//   row is reduced (max / sum / |p - q| / sign masses);
//   streaming path (any V): one 256-thread workgroup per row, element loads, the rows re-read
//   from cache per pass.
// Backward: elementwise over rows x V from the saved per-row statistics (one read of x and y,
// one write of dx).
//
// Identical draft and teacher rows go through the same instruction sequence, so their
// probabilities are bitwise equal and both the L1 loss and its subgradient are exactly zero.
#include <algorithm>

#include "common.h"

namespace aspec {
namespace {

constexpr int kStats = 8;  // per-row: mx, 1/sx, my, 1/sy, mass(p>q), mass(p<q), mass(p==q), lse_x

struct LossArgs {
  const uint16_t* x;
  const uint16_t* y;
  const int64_t* yidx;
  int64_t trows;
  const int64_t* target;
  int64_t ignore_index;
  int64_t rows, V;
  float* l1;
  float* ce;
  float* stats;
  int32_t* flags;
  int64_t* amax;  // row argmax (torch.argmax semantics), optional
  const float* g_l1;
  const float* g_ce;
  uint16_t* dx;
};

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Block-wide reduction of NVAL floats (sum or max), result broadcast to every thread.
template <int NVAL, bool MAX>
__device__ __forceinline__ void block_reduce(float (&v)[NVAL], float* scratch) {
#pragma unroll
  for (int i = 0; i < NVAL; ++i) {
    for (int off = 32; off > 0; off >>= 1) {
      const float o = __shfl_xor(v[i], off);
      v[i] = MAX ? fmaxf(v[i], o) : v[i] + o;
    }
  }
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int i = 0; i < NVAL; ++i) scratch[i * 32 + wave] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NVAL; ++i) {
    float r = scratch[i * 32];
    for (int w = 1; w < nwaves; ++w) r = MAX ? fmaxf(r, scratch[i * 32 + w]) : r + scratch[i * 32 + w];
    v[i] = r;
  }
}

__device__ __forceinline__ int64_t teacher_row(const LossArgs& a, int64_t row) {
  if (!a.yidx) return row;
  const int64_t t = a.yidx[row];
  if (t < 0 || t >= a.trows) {
    atomicOr(a.flags, 1);
    return -1;
  }
  return t;
}

__device__ __forceinline__ float bf(uint16_t v) { return bf16_to_f32(v); }

// Wave-uniform reads of kernel inputs through the scalar cache (constant address space): they
// are counted by lgkmcnt, so no wait for them also waits for the vector loads in flight.
template <typename T>
__device__ __forceinline__ T scalar_read(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}
// The bf16 at p (wave-uniform address), read as its aligned 32-bit word.
__device__ __forceinline__ float scalar_read_bf16(const uint16_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t w = scalar_read(reinterpret_cast<const uint32_t*>(a & ~static_cast<uintptr_t>(3)));
  return __uint_as_float((a & 2) ? (w & 0xffff0000u) : (w << 16));
}

// Masses of p against q: accumulates |p-q| and p split by sign(p-q) (tiled_l1.py:76-92).
__device__ __forceinline__ void l1_terms(float p, float q, float& l1, float& pos, float& neg, float& zero) {
  l1 += fabsf(p - q);
  if (p > q) pos += p;
  else if (p < q) neg += p;
  else zero += p;
}

// log2-domain exponent of a logit against its row maximum: p = exp2(v*log2e - max*log2e) / sum.
// The forward and backward kernels evaluate it with this one formula, so they classify p against
// q identically, and identical draft/teacher rows give bitwise equal probabilities.
__device__ __forceinline__ float neg_scaled_max(float m) { return -(m * kLog2e); }
__device__ __forceinline__ float scaled_exp2(float v, float nm) { return fexp2(fmaf(v, kLog2e, nm)); }

// (max, sum) pairs: sum is relative to max. A pair whose max is -inf holds 0 (all masked) or NaN
// (a NaN logit) and passes through unscaled; +inf maxima give NaN, as softmax does.
__device__ __forceinline__ void merge_max_sum(float& m, float& s, float mo, float so) {
  const float mn = fmaxf(m, mo);
  const float a = m == -INFINITY ? s : s * fexp2((m - mn) * kLog2e);
  const float b = mo == -INFINITY ? so : so * fexp2((mo - mn) * kLog2e);
  m = mn;
  s = a + b;
}

// Block-wide merge of NP (max, sum) pairs; the result is broadcast to every thread.
template <int NP>
__device__ __forceinline__ void block_max_sum(float (&m)[NP], float (&s)[NP], float* scratch) {
#pragma unroll
  for (int i = 0; i < NP; ++i)
    for (int off = 32; off > 0; off >>= 1)
      merge_max_sum(m[i], s[i], __shfl_xor(m[i], off), __shfl_xor(s[i], off));
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      scratch[(2 * i) * 32 + wave] = m[i];
      scratch[(2 * i + 1) * 32 + wave] = s[i];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float mm = scratch[(2 * i) * 32], ss = scratch[(2 * i + 1) * 32];
    for (int w = 1; w < nwaves; ++w) merge_max_sum(mm, ss, scratch[(2 * i) * 32 + w], scratch[(2 * i + 1) * 32 + w]);
    // a row of -inf (or padding only) has no softmax: NaN, as torch gives
    m[i] = mm;
    s[i] = mm == -INFINITY ? NAN : ss;
  }
}

__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

constexpr int kWalkThreads = 512;  // threads of the persistent row walk (8 waves, 2 per SIMD)
// Eight bf16 -inf: what the row walk's lanes past the end of a row load.
__device__ const uint4 kNegInfChunk = {0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u};
constexpr int kWalkWaves = kWalkThreads / 64;

// Per-thread max and exp2 values of NV chunks of eight bf16 logits (chunk j of thread t holds
// row elements (j * kWalkThreads + t) * 8 .. +7; value i of `e` is element i % 8 of chunk i / 8).
// max(a, b, c) as the hardware computes it (a NaN operand is skipped, like fmaxf). Through fmaxf
// the compiler first quiets every operand with a max of the value with itself, which more than
// doubles the cost of the row maximum; a NaN logit still reaches the row sum (and so the loss)
// through its exp.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// min(a, |b|) as one v_min_f32 with an absolute-value source modifier (fminf would first quiet
// both operands).
__device__ __forceinline__ float min_abs_raw(float a, float b) {
  float r;
  asm("v_min_f32_e64 %0, %1, |%2|" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

struct NoChunkHook {
  __device__ __forceinline__ void operator()(int) const {}
};

// `after_chunk(j)` runs once chunk j's exponentials are computed (the row walk issues a load of
// the next row there, so the loads enter the memory pipeline between VALU work).
template <int NV, typename Hook = NoChunkHook>
__device__ __forceinline__ void chunk_exps(const uint4 (&v)[NV], float (&e)[NV * 8], float& m,
                                           float& sum, const Hook& after_chunk = Hook{}) {
  m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) m = max3_raw(m, lo_bf(w[k]), hi_bf(w[k]));
  }
  const float nm = m == -INFINITY ? 0.f : neg_scaled_max(m);
  sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      e[j * 8 + 2 * k] = scaled_exp2(lo_bf(w[k]), nm);
      e[j * 8 + 2 * k + 1] = scaled_exp2(hi_bf(w[k]), nm);
      sum += e[j * 8 + 2 * k] + e[j * 8 + 2 * k + 1];
    }
    after_chunk(j);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// A (max, sum) pair's sum relative to `to` (>= its max): a pair whose max is -inf passes its sum
// (0, or NaN from a NaN logit) unscaled; a +inf max against a +inf `to` gives NaN, as softmax
// does.
__device__ __forceinline__ float sum_relative_to(float m, float s, float to) {
  return m == -INFINITY ? s : s * fexp2((m - to) * kLog2e);
}

// Merges every thread's (max, sum) pair for NP quantities: within each wave in registers, then
// across the waves through `slots` (2*NP*kWalkWaves floats, one barrier).
template <int NP>
__device__ __forceinline__ void block_merge(float (&m)[NP], float (&sm)[NP], float* slots) {
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const float mw = wave_allmax(m[i]);
    sm[i] = wave_allsum(sum_relative_to(m[i], sm[i], mw));
    m[i] = mw;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      slots[(2 * i) * kWalkWaves + wave] = m[i];
      slots[(2 * i + 1) * kWalkWaves + wave] = sm[i];
    }
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float mm = slots[(2 * i) * kWalkWaves];
#pragma unroll
    for (int w = 1; w < kWalkWaves; ++w) mm = fmaxf(mm, slots[(2 * i) * kWalkWaves + w]);
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < kWalkWaves; ++w)
      ss += sum_relative_to(slots[(2 * i) * kWalkWaves + w], slots[(2 * i + 1) * kWalkWaves + w], mm);
    m[i] = mm;
    sm[i] = mm == -INFINITY ? NAN : ss;  // a row of -inf (or padding only): NaN, as torch gives
  }
}

// Row argmax as torch.argmax defines it: the first NaN if the row has one (NaN compares above
// everything), else the first index holding the maximum M. Keys order the candidates: NaN at
// index i -> i, maximum at i -> i | 2^31, neither -> kNoKey; the row's argmax is the minimum key.
constexpr uint32_t kNoKey = 0xffffffffu;
__device__ __forceinline__ uint32_t argmax_key(float x, float M, uint32_t idx) {
  return x != x ? idx : (x == M ? (idx | 0x80000000u) : kNoKey);
}

// Block sums of NP floats and the block minimum of one key (same barrier).
template <int NP>
__device__ __forceinline__ void block_sums(float (&v)[NP], uint32_t& key, float* slots,
                                           uint32_t* key_slots) {
#pragma unroll
  for (int i = 0; i < NP; ++i) v[i] = wave_allsum(v[i]);
  key = wave_allmin(key);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int i = 0; i < NP; ++i) slots[i * kWalkWaves + wave] = v[i];
    key_slots[wave] = key;
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float r = slots[i * kWalkWaves];
#pragma unroll
    for (int w = 1; w < kWalkWaves; ++w) r += slots[i * kWalkWaves + w];
    v[i] = r;
  }
  key = key_slots[0];
#pragma unroll
  for (int w = 1; w < kWalkWaves; ++w) key = min(key, key_slots[w]);
}

// GRAD (with a teacher only): once a row's statistics are final, the walk also writes the row's
// dlogits for the objective sum_r (g_ce[r] ce[r] + g_l1[r] l1[r]) from the p and q it still holds,
// dx = p * (L1 case weight * g_l1 + g_ce) - g_ce at the target (the backward's formula), into `dx`
// (which may be the logits themselves: the row has been read by then).
template <int NV, bool ARGMAX, bool HAS_Y, bool GRAD = false>
__global__ void __launch_bounds__(kWalkThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
loss_fwd_persistent(LossArgs args) {
  static_assert(!GRAD || HAS_Y, "the fused gradient needs a teacher");
  __shared__ float merge_slots[4 * kWalkWaves];  // (max, sum) of x and y per wave
  __shared__ float sum_slots[4 * kWalkWaves];    // |p-q|, p>q, p<q masses and sum p per wave
  __shared__ uint32_t key_slots[kWalkWaves];      // argmax key per wave
  // Every field in a local: referencing the kernel argument itself from the loop would make the
  // compiler copy it to scratch.
  const uint16_t* const xbase = args.x;
  const uint16_t* const ybase = args.y;
  const int64_t* const yidx = args.yidx;
  const int64_t trows = args.trows;
  const int64_t* const target = args.target;
  const int64_t ignore = args.ignore_index;
  const int64_t rows = args.rows, V = args.V;
  float* const l1_out = args.l1;
  float* const ce_out = args.ce;
  float* const stats = args.stats;
  int32_t* const flags = args.flags;
  int64_t* const amax_out = args.amax;
  const int tid = threadIdx.x;
  constexpr bool has_y = HAS_Y;  // a compile-time teacher: every path issues the same loads
  const uint32_t nchunks = static_cast<uint32_t>(V / 8);
  uint4 nx[NV], ny[NV];
  // Chunk j of a row (j * kWalkThreads + tid). Every lane loads: a lane past the row's end reads
  // the -inf chunk, a teacher row out of range reads row 0 (its loss is NaN), and the last row of
  // a workgroup re-reads itself as its "next" row. NV is the smallest size that covers V, so only
  // chunks j >= NV/2 can reach past the row's end.
  // (global address space throughout: a select with a generic pointer would make these flat
  // loads, which LDS waits and barriers then also wait for)
  typedef const __attribute__((address_space(1))) uint4* GlobalChunk;
  auto src = [&](const uint16_t* row_base, int j) __attribute__((always_inline)) {
    const uint32_t chunk = static_cast<uint32_t>(j) * static_cast<uint32_t>(kWalkThreads) + tid;
    GlobalChunk p = (GlobalChunk)(row_base) + chunk;
    if (NV == 2 || j >= NV / 2) p = chunk < nchunks ? p : (GlobalChunk)(&kNegInfChunk);
    return (const uint4*)p;
  };
  auto load_x = [&](int j, int64_t r) __attribute__((always_inline)) { nx[j] = *src(xbase + r * V, j); };
  auto load_y = [&](int j, int64_t tr) __attribute__((always_inline)) {
    ny[j] = *src(ybase + (tr >= 0 && tr < trows ? tr : 0) * V, j);
  };
  auto teacher = [&](int64_t r) -> int64_t {  // teacher row of draft row r, -1 when out of range
    if (!has_y) return 0;
    if (!yidx) return r;
    const int64_t t = yidx[r];
    if (t < 0 || t >= trows) {
      atomicOr(flags, 1);
      return -1;
    }
    return t;
  };
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  int64_t trow = teacher(row);
  int64_t tgt = ce_out ? target[row] : ignore;
#pragma unroll
  for (int j = 0; j < NV; ++j) load_x(j, row);
  if (has_y) {
#pragma unroll
    for (int j = 0; j < NV; ++j) load_y(j, trow);
  }
  while (row < rows) {
    // The next row's teacher index and target: loaded here, first used after the next row's draft
    // logits have been requested (so waiting for them waits for nothing else).
    const int64_t next = row + gridDim.x;
    const int64_t nsafe = next < rows ? next : row;
    const int64_t tidx_n = has_y && yidx ? scalar_read(yidx + nsafe) : nsafe;
    const int64_t tgt_n = ce_out ? scalar_read(target + nsafe) : ignore;
    // the CE target logit (from cache: the row has just been read)
    const bool tgt_ok = tgt != ignore && tgt >= 0 && tgt < V;
    const float target_logit = tgt_ok ? scalar_read_bf16(xbase + row * V + tgt) : 0.f;
    float ex[NV * 8], ey[NV * 8];
    float m[2], sm[2];
    chunk_exps<NV>(nx, ex, m[0], sm[0]);
    m[1] = -INFINITY;
    sm[1] = 0.f;
    // The next row's draft logits stream in while the teacher's exponentials are computed (one
    // chunk per step, into the registers chunk_exps has just consumed), its teacher logits during
    // the L1 masses below.
    if (has_y) {
      chunk_exps<NV>(ny, ey, m[1], sm[1], [&](int j) __attribute__((always_inline)) { load_x(j, nsafe); });
    } else {
#pragma unroll
      for (int j = 0; j < NV; ++j) load_x(j, nsafe);
    }
    const float mx_local = m[0], my_local = m[1], sx_local = sm[0];
    block_merge<2>(m, sm, merge_slots);
    uint32_t key = kNoKey;
    if (ARGMAX) {
      const float M = m[0];
      if (fabsf(M) >= 0x1p-14f && M < INFINITY && sm[0] == sm[0]) {
        // A finite row without NaN whose maximum is not tiny: a thread holding M finds its first
        // maximal element among its exp values, which hold exp2(x log2e - M log2e) (chunk_exps).
        // The maximum gives exactly `emax` (same expression), and any other bf16 logit differs
        // from M by at least |M| 2^-8, far above the rounding of M log2e, so it never does.
        if (mx_local == M) {
          const float emax = scaled_exp2(M, neg_scaled_max(M));
          uint32_t i0 = 0;  // first exp value equal to emax (immediates: nothing hoisted per value)
#pragma unroll
          for (int i = NV * 8 - 1; i >= 0; --i) i0 = ex[i] == emax ? static_cast<uint32_t>(i) : i0;
          key = ((((i0 >> 3) * kWalkThreads + tid) << 3) + (i0 & 7)) | 0x80000000u;
        }
      } else {
        // a NaN, an infinity, an all -inf row or a tiny maximum: rescan the (cache-resident) row
        const uint16_t* xr = xbase + row * V;
        for (int64_t i = tid; i < V; i += kWalkThreads)
          key = min(key, argmax_key(bf(xr[i]), M, static_cast<uint32_t>(i)));
      }
    }
    // p = e * 2^((m_local - M) log2e) / S per thread (0 for threads whose chunk is all -inf)
    const float cx = (mx_local == -INFINITY ? 0.f : fexp2((mx_local - m[0]) * kLog2e)) / sm[0];
    const float cy = (my_local == -INFINITY ? 0.f : fexp2((my_local - m[1]) * kLog2e)) / sm[1];
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // |p-q|, mass p>q, mass p<q, sum p
    int64_t trow_n = 0;
    if (has_y) {
      trow_n = tidx_n;
      if (yidx && next < rows && (trow_n < 0 || trow_n >= trows)) {
        if (tid == 0) atomicOr(flags, 1);
        trow_n = -1;
      }
      // Every chunk but the last (the only one that can reach past the row's end): |p - q| and,
      // unless the chunk holds an exact tie, the signed mass S = sum copysign(p, p - q), seven VALU
      // operations per element; then, with T = sum p over those chunks, mass(p > q) = (T + S) / 2
      // and mass(p < q) = (T - S) / 2. A chunk with a tie (identical rows, both logits masked)
      // and the last chunk count their masses element by element, so ties keep their own mass
      // exactly (identical rows give exactly zero masses and gradient).
      float sgn = 0.f, exact_sum = 0.f;
      bool any_fast = false;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        float pj[8], dj[8];
        float mj = INFINITY;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          pj[k] = ex[j * 8 + k] * cx;
          dj[k] = pj[k] - ey[j * 8 + k] * cy;
          acc[0] += fabsf(dj[k]);
          mj = min_abs_raw(mj, dj[k]);
        }
        if (j < NV - 1 && mj != 0.f) {
          any_fast = true;
#pragma unroll
          for (int k = 0; k < 8; ++k) sgn += copysignf(pj[k], dj[k]);
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            acc[1] += dj[k] > 0.f ? pj[k] : 0.f;
            acc[2] += dj[k] < 0.f ? pj[k] : 0.f;
            exact_sum += pj[k];
          }
        }
        if constexpr (!GRAD) load_y(j, trow_n);  // GRAD: after this chunk's dlogits (below)
        __builtin_amdgcn_sched_barrier(0);
      }
      const float total = cx * sx_local;
      if (any_fast) {
        const float t = total - exact_sum;
        acc[1] += 0.5f * (t + sgn);
        acc[2] += 0.5f * (t - sgn);
      }
      acc[3] = total;
    }
    block_sums<4>(acc, key, sum_slots, key_slots);
    if constexpr (GRAD) {
      // the row's objective weights (wave-uniform) and the three L1 case weights (the backward's
      // centered terms, tiled_l1.py:107-127)
      const float wl1 = trow >= 0 ? scalar_read(args.g_l1 + row) : NAN;
      const float wce = tgt != ignore ? scalar_read(args.g_ce + row) : 0.f;
      const float pos = acc[1], neg = acc[2], zero = acc[3] - acc[1] - acc[2];
      const float k_gt = (2.f * neg + zero) * wl1 + wce;
      const float k_lt = (-2.f * pos - zero) * wl1 + wce;
      const float k_eq = (neg - pos) * wl1 + wce;
      uint16_t* const drow = args.dx + row * V;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const uint32_t chunk = static_cast<uint32_t>(j) * static_cast<uint32_t>(kWalkThreads) + tid;
        float d[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float pv = ex[j * 8 + k] * cx, qv = ey[j * 8 + k] * cy;
          d[k] = pv * (pv > qv ? k_gt : (pv < qv ? k_lt : k_eq));
        }
        // the CE target: chunk tgt / 8 belongs to thread (tgt / 8) % kWalkThreads at step
        // (tgt / 8) / kWalkThreads (all wave-uniform but the thread)
        if (tgt_ok && (tgt >> 3) / kWalkThreads == j && static_cast<int64_t>(tid) == (tgt >> 3) % kWalkThreads) {
          switch (static_cast<int>(tgt & 7)) {
            case 0: d[0] -= wce; break;
            case 1: d[1] -= wce; break;
            case 2: d[2] -= wce; break;
            case 3: d[3] -= wce; break;
            case 4: d[4] -= wce; break;
            case 5: d[5] -= wce; break;
            case 6: d[6] -= wce; break;
            default: d[7] -= wce; break;
          }
        }
        if (chunk < nchunks)
          reinterpret_cast<uint4*>(drow)[chunk] =
              make_uint4(pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3]), pack_bf16x2(d[4], d[5]),
                         pack_bf16x2(d[6], d[7]));
        // the next row's teacher chunk, into registers this row no longer needs
        load_y(j, trow_n);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (tid == 0) {
      if (ARGMAX) amax_out[row] = static_cast<int64_t>(key & 0x7fffffffu);
      const float lse = logf(sm[0]) + m[0];
      float* st = stats + row * kStats;
      st[0] = m[0]; st[1] = 1.f / sm[0]; st[2] = m[1]; st[3] = 1.f / sm[1];
      st[4] = acc[1]; st[5] = acc[2]; st[6] = acc[3] - acc[1] - acc[2]; st[7] = lse;
      if (l1_out) l1_out[row] = (has_y && trow >= 0) ? acc[0] : NAN;
      if (ce_out) {
        float v = 0.f;
        if (tgt != ignore) {
          if (!tgt_ok) { atomicOr(flags, 2); v = NAN; }
          else v = lse - target_logit;
        }
        ce_out[row] = v;
      }
    }
    row = next;
    trow = trow_n;
    tgt = tgt_n;
  }
}

// Any vocabulary size: element loads, three passes over the (cache-resident) row.
__global__ void __launch_bounds__(256) loss_fwd_streaming(LossArgs a) {
  __shared__ float scratch[4 * 32];
  const int64_t row = blockIdx.x;
  const bool has_y = a.y != nullptr;
  const int64_t trow = has_y ? teacher_row(a, row) : 0;
  const uint16_t* xr = a.x + row * a.V;
  const uint16_t* yr = has_y && trow >= 0 ? a.y + trow * a.V : nullptr;
  float m[2] = {-INFINITY, -INFINITY};
  for (int64_t i = threadIdx.x; i < a.V; i += blockDim.x) {
    m[0] = fmaxf(m[0], bf(xr[i]));
    if (yr) m[1] = fmaxf(m[1], bf(yr[i]));
  }
  float s[2] = {0.f, 0.f};
  {
    const float nx = m[0] == -INFINITY ? 0.f : neg_scaled_max(m[0]);
    const float ny = m[1] == -INFINITY ? 0.f : neg_scaled_max(m[1]);
    for (int64_t i = threadIdx.x; i < a.V; i += blockDim.x) {
      s[0] += scaled_exp2(bf(xr[i]), nx);
      if (yr) s[1] += scaled_exp2(bf(yr[i]), ny);
    }
  }
  block_max_sum<2>(m, s, scratch);
  if (a.amax) {  // first NaN, else first maximum (torch.argmax)
    uint32_t key = kNoKey;
    for (int64_t i = threadIdx.x; i < a.V; i += blockDim.x)
      key = min(key, argmax_key(bf(xr[i]), m[0], static_cast<uint32_t>(i)));
    for (int off = 32; off > 0; off >>= 1)
      key = min(key, static_cast<uint32_t>(__shfl_xor(static_cast<int>(key), off)));
    __shared__ uint32_t keys[8];
    if ((threadIdx.x & 63) == 0) keys[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) key = min(key, keys[w]);
      a.amax[row] = static_cast<int64_t>(key & 0x7fffffffu);
    }
  }
  const float nmx = neg_scaled_max(m[0]), nmy = neg_scaled_max(m[1]);
  const float ix = 1.f / s[0], iy = 1.f / s[1];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (has_y) {
    for (int64_t i = threadIdx.x; i < a.V; i += blockDim.x) {
      const float p = scaled_exp2(bf(xr[i]), nmx) * ix;
      const float q = yr ? scaled_exp2(bf(yr[i]), nmy) * iy : NAN;
      l1_terms(p, q, acc[0], acc[1], acc[2], acc[3]);
    }
    block_reduce<4, false>(acc, scratch);
  }
  if (threadIdx.x == 0) {
    const float lse = logf(s[0]) + m[0];
    float* st = a.stats + row * kStats;
    st[0] = m[0]; st[1] = ix; st[2] = m[1]; st[3] = iy;
    st[4] = acc[1]; st[5] = acc[2]; st[6] = acc[3]; st[7] = lse;
    if (a.l1) a.l1[row] = (has_y && trow >= 0) ? acc[0] : NAN;
    if (a.ce) {
      const int64_t t = a.target[row];
      float v = 0.f;
      if (t != a.ignore_index) {
        if (t < 0 || t >= a.V) { atomicOr(a.flags, 2); v = NAN; }
        else v = lse - bf(xr[t]);
      }
      a.ce[row] = v;
    }
  }
}

// dx = g_ce * (p - onehot(t)) + g_l1 * p * centered  (tiled_l1.py:107-127 for the L1 part).
__device__ __forceinline__ float grad_elem(float x, float y, const float* st, float gl1, float gce,
                                           bool is_target, bool has_y) {
  const float p = scaled_exp2(x, neg_scaled_max(st[0])) * st[1];
  float d = 0.f;
  if (has_y) {
    const float q = scaled_exp2(y, neg_scaled_max(st[2])) * st[3];
    const float pos = st[4], neg = st[5], zero = st[6];
    const float centered = p > q ? 2.f * neg + zero : (p < q ? -2.f * pos - zero : neg - pos);
    d = p * centered * gl1;
  }
  if (gce != 0.f) d += gce * (p - (is_target ? 1.f : 0.f));
  return d;
}

// Vectorised path (V % 8 == 0): each workgroup pass covers 256 consecutive chunks of eight logits
// of one row, so the row's statistics, upstream gradients, target and teacher index are
// wave-uniform and read through the scalar cache; only the logits and dx use the vector memory
// path.
constexpr int kBwdThreads = 256;

__global__ void __launch_bounds__(kBwdThreads) loss_bwd_rows_kernel(LossArgs a) {
  const int64_t per_row = a.V / 8;
  const int64_t segs_per_row = (per_row + kBwdThreads - 1) / kBwdThreads;
  const int64_t segs = a.rows * segs_per_row;
  const bool has_y = a.y != nullptr;
  for (int64_t seg = blockIdx.x; seg < segs; seg += gridDim.x) {
    const int64_t row = seg / segs_per_row;
    const int64_t chunk = (seg - row * segs_per_row) * kBwdThreads + threadIdx.x;
    float st[kStats];
#pragma unroll
    for (int i = 0; i < kStats; ++i) st[i] = scalar_read(a.stats + row * kStats + i);
    const float gl1 = (has_y && a.g_l1) ? scalar_read(a.g_l1 + row) : 0.f;
    float gce = 0.f;
    int64_t tgt = -1;
    if (a.g_ce) {
      tgt = scalar_read(a.target + row);
      gce = tgt == a.ignore_index ? 0.f : scalar_read(a.g_ce + row);
    }
    int64_t trow = 0;
    if (has_y) {
      trow = a.yidx ? scalar_read(a.yidx + row) : row;
      if (trow < 0 || trow >= a.trows) trow = -1;
    }
    if (chunk >= per_row) continue;
    // dx = p * (L1 weight of the element's case + g_ce) - g_ce at the target, p = e_x / S_x with
    // e = exp2(v log2e - max log2e) (scaled_exp2, as grad_elem). Per row: the three case weights
    // times 1/S_x, and r = (1/S_y) / (1/S_x), so p against q is e_x against e_y * r (identical rows:
    // r = 1 and e_x == e_y, the p == q case).
    const float nmx = neg_scaled_max(st[0]), nmy = neg_scaled_max(st[2]);
    const float pos = st[4], neg = st[5], zero = st[6];
    const float k_gt = st[1] * ((2.f * neg + zero) * gl1 + gce);
    const float k_lt = st[1] * ((-2.f * pos - zero) * gl1 + gce);
    const float k_eq = st[1] * ((neg - pos) * gl1 + gce);
    const float k_ce = st[1] * gce;  // no teacher: the CE part alone
    const float r = st[3] / st[1];
    const int64_t col0 = chunk * 8;
    const uint16_t* xr = a.x + row * a.V;
    const uint16_t* yr = (has_y && trow >= 0) ? a.y + trow * a.V : nullptr;
    const uint4 xs = *reinterpret_cast<const uint4*>(xr + col0);
    const uint4 ys = yr ? *reinterpret_cast<const uint4*>(yr + col0) : make_uint4(0, 0, 0, 0);
    const uint32_t xw[4] = {xs.x, xs.y, xs.z, xs.w};
    const uint32_t yw[4] = {ys.x, ys.y, ys.z, ys.w};
    float d[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = (e & 1) ? __uint_as_float(xw[e >> 1] & 0xffff0000u) : __uint_as_float(xw[e >> 1] << 16);
      const float ex = scaled_exp2(x, nmx);
      float k = k_ce;
      if (has_y) {
        if (yr) {
          const float y = (e & 1) ? __uint_as_float(yw[e >> 1] & 0xffff0000u) : __uint_as_float(yw[e >> 1] << 16);
          const float qs = scaled_exp2(y, nmy) * r;
          k = ex > qs ? k_gt : (ex < qs ? k_lt : k_eq);
        } else {
          k = NAN;  // teacher row out of range: NaN, as grad_elem gives
        }
      }
      d[e] = ex * k;
    }
    // the CE target column (one lane of the row)
    if (gce != 0.f && tgt >= col0 && tgt < col0 + 8) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (col0 + e == tgt) d[e] -= gce;
    }
    uint32_t out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = pack_bf16x2(d[2 * e], d[2 * e + 1]);
    *reinterpret_cast<uint4*>(a.dx + row * a.V + col0) = make_uint4(out[0], out[1], out[2], out[3]);
  }
}

template <bool VEC>
__global__ void __launch_bounds__(256) loss_bwd_kernel(LossArgs a) {
  const int64_t per_row = VEC ? a.V / 8 : a.V;
  const int64_t total = a.rows * per_row;
  const bool has_y = a.y != nullptr;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = t / per_row;
    const int64_t col0 = (t - row * per_row) * (VEC ? 8 : 1);
    float st[kStats];
#pragma unroll
    for (int i = 0; i < kStats; ++i) st[i] = a.stats[row * kStats + i];
    const float gl1 = (has_y && a.g_l1) ? a.g_l1[row] : 0.f;
    float gce = 0.f;
    int64_t tgt = -1;
    if (a.g_ce) {
      tgt = a.target[row];
      gce = tgt == a.ignore_index ? 0.f : a.g_ce[row];
    }
    int64_t trow = 0;
    if (has_y) {
      trow = a.yidx ? a.yidx[row] : row;
      if (trow < 0 || trow >= a.trows) trow = -1;
    }
    const uint16_t* xr = a.x + row * a.V;
    const uint16_t* yr = (has_y && trow >= 0) ? a.y + trow * a.V : nullptr;
    if (VEC) {
      const uint4 xs = *reinterpret_cast<const uint4*>(xr + col0);
      const uint4 ys = yr ? *reinterpret_cast<const uint4*>(yr + col0) : make_uint4(0, 0, 0, 0);
      const uint32_t xw[4] = {xs.x, xs.y, xs.z, xs.w};
      const uint32_t yw[4] = {ys.x, ys.y, ys.z, ys.w};
      uint32_t out[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y0 = yr ? __uint_as_float(yw[e] << 16) : NAN;
        const float y1 = yr ? __uint_as_float(yw[e] & 0xffff0000u) : NAN;
        const float d0 = grad_elem(__uint_as_float(xw[e] << 16), y0, st, gl1, gce, col0 + 2 * e == tgt, has_y);
        const float d1 = grad_elem(__uint_as_float(xw[e] & 0xffff0000u), y1, st, gl1, gce, col0 + 2 * e + 1 == tgt, has_y);
        out[e] = pack_bf16x2(d0, d1);
      }
      *reinterpret_cast<uint4*>(a.dx + row * a.V + col0) = make_uint4(out[0], out[1], out[2], out[3]);
    } else {
      const float y = yr ? bf(yr[col0]) : NAN;
      const float d = grad_elem(bf(xr[col0]), y, st, gl1, gce, col0 == tgt, has_y);
      a.dx[row * a.V + col0] = f32_to_bf16_bits(d);
    }
  }
}

template <int NV>
void launch_walk(const LossArgs& a, dim3 walk, dim3 block, hipStream_t s) {
  if (a.dx) {  // the fused forward + dlogits (teacher present, checked by the entry point)
    if (a.amax) hipLaunchKernelGGL((loss_fwd_persistent<NV, true, true, true>), walk, block, 0, s, a);
    else hipLaunchKernelGGL((loss_fwd_persistent<NV, false, true, true>), walk, block, 0, s, a);
    return;
  }
  if (a.y) {
    if (a.amax) hipLaunchKernelGGL((loss_fwd_persistent<NV, true, true>), walk, block, 0, s, a);
    else hipLaunchKernelGGL((loss_fwd_persistent<NV, false, true>), walk, block, 0, s, a);
  } else {
    if (a.amax) hipLaunchKernelGGL((loss_fwd_persistent<NV, true, false>), walk, block, 0, s, a);
    else hipLaunchKernelGGL((loss_fwd_persistent<NV, false, false>), walk, block, 0, s, a);
  }
}

int launch_fwd(const LossArgs& a, hipStream_t s) {
  const bool vec = a.V % 8 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                   (!a.y || (reinterpret_cast<uintptr_t>(a.y) & 15) == 0);
  const dim3 grid(static_cast<uint32_t>(a.rows));
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return set_error(ASPEC_ERR_RUNTIME, "cannot query the GPU's compute-unit count");
  const dim3 walk(static_cast<uint32_t>(std::min<int64_t>(a.rows, cus)));
  const dim3 block(kWalkThreads);
  if (a.dx && !(vec && a.V <= kWalkThreads * 8 * 8 && (reinterpret_cast<uintptr_t>(a.dx) & 15) == 0))
    return set_error(ASPEC_ERR_UNSUPPORTED, "the fused loss forward + dlogits needs V %% 8 == 0, V <= %d "
                     "and 16-byte aligned rows", kWalkThreads * 8 * 8);
  if (vec && a.V <= kWalkThreads * 8 * 2) {
    launch_walk<2>(a, walk, block, s);
  } else if (vec && a.V <= kWalkThreads * 8 * 4) {
    launch_walk<4>(a, walk, block, s);
  } else if (vec && a.V <= kWalkThreads * 8 * 8) {
    launch_walk<8>(a, walk, block, s);
  } else {
    hipLaunchKernelGGL(loss_fwd_streaming, grid, dim3(256), 0, s, a);
  }
  return check_launch("loss forward");
}

int launch_bwd(const LossArgs& a, hipStream_t s) {
  const bool vec = a.V % 8 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                   (!a.y || (reinterpret_cast<uintptr_t>(a.y) & 15) == 0) &&
                   (reinterpret_cast<uintptr_t>(a.dx) & 15) == 0;
  const int64_t work = a.rows * (vec ? a.V / 8 : a.V);
  const int64_t blocks = std::min<int64_t>((work + 255) / 256, 256 * 64);
  if (vec) {
    const int64_t segs = a.rows * ((a.V / 8 + kBwdThreads - 1) / kBwdThreads);
    const int64_t grid = std::min<int64_t>(segs, 256 * 64);
    hipLaunchKernelGGL(loss_bwd_rows_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kBwdThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL(loss_bwd_kernel<false>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, a);
  }
  return check_launch("loss backward");
}

// Two bf16 in one word, each times s: fp32 product, one round to nearest even.
__device__ __forceinline__ uint32_t scale_bf16_pair(uint32_t w, float s) {
  return pack_bf16x2(__uint_as_float(w << 16) * s, __uint_as_float(w & 0xffff0000u) * s);
}

// x *= s in place over n bf16 values, s read on the device. When s == 1 every product equals its
// input bit for bit, so each workgroup returns before touching x (the usual upstream gradient of a
// loss: the multiply costs a launch instead of a pass over x). n8 16-byte groups, then the tail.
__global__ void __launch_bounds__(256) scale_bf16_kernel(uint16_t* x, int64_t n, int64_t n8,
                                                         const float* scalar) {
  const float s = scalar_read(scalar);
  if (s == 1.0f) return;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  uint4* v = reinterpret_cast<uint4*>(x);
  for (int64_t i = first; i < n8; i += stride) {
    uint4 w = v[i];
    w.x = scale_bf16_pair(w.x, s);
    w.y = scale_bf16_pair(w.y, s);
    w.z = scale_bf16_pair(w.z, s);
    w.w = scale_bf16_pair(w.w, s);
    v[i] = w;
  }
  for (int64_t i = n8 * 8 + first; i < n; i += stride)
    x[i] = f32_to_bf16_bits(bf16_to_f32(x[i]) * s);
}

int check_common(int64_t rows, int64_t V, const void* x) {
  if (rows <= 0 || V <= 0 || !x)
    return set_error(ASPEC_ERR_INVALID, "loss kernels require nonempty logits with a vocabulary dimension");
  return ASPEC_OK;
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_loss_stats_floats(void) { return kStats; }

extern "C" int aspec_ce_l1_argmax_fwd(const void* logits, const void* teacher,
                                      const int64_t* teacher_index, int64_t teacher_rows,
                                      const int64_t* targets, int64_t ignore_index, int64_t rows,
                                      int64_t vocab, float* l1_out, float* ce_out, int64_t* argmax_out,
                                      float* stats, int32_t* status_flags, void* stream) {
  int rc = check_common(rows, vocab, logits);
  if (rc) return rc;
  if (!stats || !status_flags) return set_error(ASPEC_ERR_INVALID, "stats and status buffers are required");
  if (l1_out && !teacher) return set_error(ASPEC_ERR_INVALID, "L1 needs teacher logits");
  if (ce_out && !targets) return set_error(ASPEC_ERR_INVALID, "cross-entropy needs targets");
  if (teacher_index && teacher_rows <= 0) return set_error(ASPEC_ERR_INVALID, "indexed teacher table is empty");
  LossArgs a = {};
  a.x = static_cast<const uint16_t*>(logits);
  a.y = static_cast<const uint16_t*>(teacher);
  a.yidx = teacher_index;
  a.trows = teacher_index ? teacher_rows : rows;
  a.target = targets;
  a.ignore_index = ignore_index;
  a.rows = rows;
  a.V = vocab;
  a.l1 = l1_out;
  a.ce = ce_out;
  a.stats = stats;
  a.flags = status_flags;
  a.amax = argmax_out;
  if (argmax_out && vocab > 0x7fffffffLL)
    return set_error(ASPEC_ERR_UNSUPPORTED, "argmax needs a vocabulary below 2^31");
  return launch_fwd(a, static_cast<hipStream_t>(stream));
}

extern "C" int aspec_ce_l1_fused_fwd_bwd(const void* logits, const void* teacher,
                                          const int64_t* teacher_index, int64_t teacher_rows,
                                          const int64_t* targets, int64_t ignore_index, int64_t rows,
                                          int64_t vocab, const float* grad_ce, const float* grad_l1,
                                          float* l1_out, float* ce_out, int64_t* argmax_out,
                                          float* stats, void* grad_logits, int32_t* status_flags,
                                          void* stream) {
  int rc = check_common(rows, vocab, logits);
  if (rc) return rc;
  if (!teacher || !targets || !grad_ce || !grad_l1 || !grad_logits || !stats || !status_flags || !l1_out || !ce_out)
    return set_error(ASPEC_ERR_INVALID, "the fused loss needs teacher logits, targets, both per-row "
                     "gradients, outputs, stats, a status buffer and a dlogits buffer");
  if (teacher_index && teacher_rows <= 0) return set_error(ASPEC_ERR_INVALID, "indexed teacher table is empty");
  if (argmax_out && vocab > 0x7fffffffLL)
    return set_error(ASPEC_ERR_UNSUPPORTED, "argmax needs a vocabulary below 2^31");
  LossArgs a = {};
  a.x = static_cast<const uint16_t*>(logits);
  a.y = static_cast<const uint16_t*>(teacher);
  a.yidx = teacher_index;
  a.trows = teacher_index ? teacher_rows : rows;
  a.target = targets;
  a.ignore_index = ignore_index;
  a.rows = rows;
  a.V = vocab;
  a.l1 = l1_out;
  a.ce = ce_out;
  a.stats = stats;
  a.flags = status_flags;
  a.amax = argmax_out;
  a.g_ce = grad_ce;
  a.g_l1 = grad_l1;
  a.dx = static_cast<uint16_t*>(grad_logits);
  return launch_fwd(a, static_cast<hipStream_t>(stream));
}

extern "C" int aspec_scale_bf16_by_device_scalar(void* x, int64_t n, const float* scalar,
                                                  void* stream) {
  if (n < 0 || (n > 0 && (!x || !scalar)))
    return set_error(ASPEC_ERR_INVALID, "scaling needs a buffer, a size >= 0 and a device scalar");
  if (n == 0) return ASPEC_OK;
  const int64_t n8 = (reinterpret_cast<uintptr_t>(x) & 15) == 0 ? n / 8 : 0;
  const int64_t work = std::max<int64_t>(n8, n - n8 * 8);
  const int64_t grid = std::min<int64_t>((work + 255) / 256, 1024);
  hipLaunchKernelGGL(scale_bf16_kernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t*>(x), n, n8, scalar);
  return check_launch("bf16 scale");
}

extern "C" int aspec_ce_l1_fwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                               int64_t teacher_rows, const int64_t* targets, int64_t ignore_index,
                               int64_t rows, int64_t vocab, float* l1_out, float* ce_out,
                               float* stats, int32_t* status_flags, void* stream) {
  return aspec_ce_l1_argmax_fwd(logits, teacher, teacher_index, teacher_rows, targets, ignore_index,
                                rows, vocab, l1_out, ce_out, nullptr, stats, status_flags, stream);
}

extern "C" int aspec_ce_l1_bwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                               int64_t teacher_rows, const int64_t* targets, int64_t ignore_index,
                               int64_t rows, int64_t vocab, const float* stats,
                               const float* grad_l1, const float* grad_ce, void* grad_logits,
                               void* stream) {
  int rc = check_common(rows, vocab, logits);
  if (rc) return rc;
  if (!stats || !grad_logits) return set_error(ASPEC_ERR_INVALID, "stats and gradient buffers are required");
  if (grad_l1 && !teacher) return set_error(ASPEC_ERR_INVALID, "L1 gradient needs teacher logits");
  if (grad_ce && !targets) return set_error(ASPEC_ERR_INVALID, "cross-entropy gradient needs targets");
  LossArgs a = {};
  a.x = static_cast<const uint16_t*>(logits);
  a.y = grad_l1 ? static_cast<const uint16_t*>(teacher) : nullptr;
  a.yidx = teacher_index;
  a.trows = teacher_index ? teacher_rows : rows;
  a.target = targets;
  a.ignore_index = ignore_index;
  a.rows = rows;
  a.V = vocab;
  a.stats = const_cast<float*>(stats);
  a.g_l1 = grad_l1;
  a.g_ce = grad_ce;
  a.dx = static_cast<uint16_t*>(grad_logits);
  return launch_bwd(a, static_cast<hipStream_t>(stream));
}
