// Sampled L1: the DSpark L1 term between temperature / top-p / top-k filtered draft and teacher
// distributions (aspec/models/ops/loss.py:57-89), and the filtered logits themselves.
//
// Per row and side (draft: `draft_sampling`, teacher: `target_sampling`):
//   scaled = temperature != 1 ? (x - max x) * (1/T) : x            (fp32, x the bf16 logit)
//   order  = scaled descending, ties by token index (a stable sort)
//   keep   = rank < top_k (0 < top_k < V)  and  mass before the token <= top_p (top_p < 1),
//            the mass from softmax(scaled) over the full row
//   p      = softmax(scaled) over the kept tokens, 0 elsewhere;  l1 = sum |p_draft - p_teacher|.
//
// One 512-thread workgroup owns a row; the row lives in registers as packed bf16 (NV chunks of
// eight per thread, up to 98304 tokens; longer rows are read again from global memory on each
// pass) and nothing is sorted. scaled is a non-decreasing function of the bf16 value,
// so the top-p boundary is the smallest 16-bit bf16 key whose strictly-greater mass is <= top_p:
// a binary search of 16 block reductions over the key space (top-k: the same over counts). One
// pass then forms the boundary's tie group in scaled values (a temperature can merge neighbouring
// bf16 values into one fp32 value), the kept count within it follows from the group's mass per
// token, and, when the group is cut, a search over token indices finds the last kept token. A
// token is kept iff its scaled key is above the boundary key, or equal and its index <= last.
// Masses are fp32 per token, summed in fp64 in a fixed order (deterministic).
#include <cmath>

#include "common.h"

namespace aspec {
namespace {

constexpr int kSampThreads = 512;
constexpr int kSampWaves = kSampThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr uint32_t kNegInfBits = 0xff80u;  // bf16 -inf: the padding of a row's tail

// per-row, per-side record (8 words); the sampled-L1 row holds draft, teacher, then the masses
constexpr int kSideWords = 8;
constexpr int kL1Words = 24;
constexpr uint32_t kFlagTemp = 1, kFlagNaN = 2, kFlagAll = 4;

struct SideParams {
  float rcp_t;   // 1/T in fp32 (1 without a temperature)
  float top_p;   // fp32, as the reference compares its fp32 cumulative mass
  int64_t top_k;
  int temp, use_p, use_k;
};

struct SideStats {
  float m;        // row max of the logits
  float rcp_t;
  uint32_t okey;  // boundary key of the scaled values
  int32_t last;   // last kept token index among the boundary ties
  float zinv;     // 1 / sum over kept tokens of exp(scaled - max scaled)
  uint32_t flags;
  int32_t nmax;   // tokens equal to the max (the max's gradient is shared among them)
  uint32_t pad;
};

struct SampledArgs {
  const uint16_t* x;
  const uint16_t* y;
  const int64_t* yidx;
  int64_t trows, rows, V;
  SideParams px, py;
  float* out;          // sampling_logits: fp32 [rows][V]
  const float* gout;   // sampling_logits backward: fp32 [rows][V]
  float* l1;
  float* stats;
  const float* g_l1;
  uint16_t* dx;
  int32_t* flags;
};

__device__ __forceinline__ float bf16f(uint32_t h) { return __uint_as_float(h << 16); }

// ordered key of an fp32 value (-0 equals +0, as in a sort's comparisons)
__device__ __forceinline__ uint32_t ord_key(float o) {
  uint32_t b = __float_as_uint(o);
  if ((b << 1) == 0) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// ordered 16-bit key of a bf16 value, and back
__device__ __forceinline__ uint32_t x_key(uint32_t h) {
  if ((h & 0x7fffu) == 0) h = 0;
  return (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
}
__device__ __forceinline__ uint32_t x_bits_of_key(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
}

struct RowCtx {
  float m, rcp_t;
  bool temp;
};
// exp(scaled - max scaled) and the sort value of a logit; one expression everywhere, so the
// forward, the backward and both sides of a row agree bit for bit
__device__ __forceinline__ float u_of(float x, const RowCtx& c) { return (x - c.m) * c.rcp_t; }
__device__ __forceinline__ float e_of(float x, const RowCtx& c) {
  return __builtin_amdgcn_exp2f(u_of(x, c) * kLog2e);
}
__device__ __forceinline__ float ord_of(float x, const RowCtx& c) { return c.temp ? u_of(x, c) : x; }

__device__ __forceinline__ RowCtx ctx_of(const SideStats& s) {
  return RowCtx{s.m, s.rcp_t, (s.flags & kFlagTemp) != 0};
}
// branch-free: evaluated for every token of a pass
__device__ __forceinline__ bool kept(const SideStats& s, uint32_t okey, int64_t idx) {
  return ((s.flags & kFlagAll) != 0) | (okey > s.okey) | ((okey == s.okey) & (idx <= s.last));
}
// probability of a token after filtering (0 outside the support)
__device__ __forceinline__ float prob(const SideStats& s, uint32_t h, int64_t idx) {
  const RowCtx c = ctx_of(s);
  const float x = bf16f(h);
  return kept(s, ord_key(ord_of(x, c)), idx) ? e_of(x, c) * s.zinv : 0.0f;
}

// ---- block reductions over the 8 waves, fixed order, every thread gets the total ---------------
struct Red {
  double slot[2][kSampWaves];
};

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// A value every lane holds alike, moved to scalar registers (the row's statistics and search
// bounds then take no vector registers beside the row itself).
__device__ __forceinline__ double uniform(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Two slot sets used alternately: the barrier of the call in between separates the reads of one
// call from the writes of the call after next. Lane l of every 8-lane group reads wave l's slot
// and a butterfly over the group adds them (a fixed pairing: every lane gets the same total).
__device__ __forceinline__ double block_total(double wave_value, Red& r, int& ph) {
  double* slot = r.slot[ph];
  ph ^= 1;
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = wave_value;
  __syncthreads();
  double s = slot[threadIdx.x & (kSampWaves - 1)];
#pragma unroll
  for (int o = kSampWaves / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, kSampWaves);
  return uniform(s);
}
__device__ __forceinline__ double block_sum(double v, Red& r, int& ph) {
  return block_total(wave_sum_d(v), r, ph);
}
__device__ __forceinline__ int64_t block_count(uint32_t v, Red& r, int& ph) {
  return static_cast<int64_t>(block_total(static_cast<double>(wave_sum_u(v)), r, ph));
}
__device__ __forceinline__ float block_max(float v, Red& r, int& ph) {
  double* slot = r.slot[ph];
  ph ^= 1;
  v = wave_max_f(v);
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = static_cast<double>(v);
  __syncthreads();
  double s = slot[threadIdx.x & (kSampWaves - 1)];
#pragma unroll
  for (int o = kSampWaves / 2; o > 0; o >>= 1) s = fmax(s, __shfl_xor(s, o, kSampWaves));
  return static_cast<float>(uniform(s));
}

// ---- rows -------------------------------------------------------------------------------------
// Chunk c of thread t is tokens (c * 512 + t) * 8 .. + 7; tokens past V read as bf16 -inf.
__device__ __forceinline__ uint4 load_chunk(const uint16_t* row, int64_t V, bool vec, int64_t base) {
  if (vec && base < V) return *reinterpret_cast<const uint4*>(row + base);
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = base + 2 * k < V ? row[base + 2 * k] : kNegInfBits;
    const uint32_t hi = base + 2 * k + 1 < V ? row[base + 2 * k + 1] : kNegInfBits;
    w[k] = lo | (hi << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ int32_t opaque_t8() {
  int32_t t8 = static_cast<int32_t>(threadIdx.x) * 8;
  asm volatile("" : "+v"(t8));
  return t8;
}
__device__ __forceinline__ uint32_t half_of(const uint32_t (&w)[4], int j) {
  return (j & 1) ? w[j >> 1] >> 16 : w[j >> 1] & 0xffffu;
}

// A row held in registers (NV chunks of packed bf16 per thread: up to 98304 tokens). Each pass
// runs the words through an empty asm in place (no copy, no instruction) and rebuilds the token
// index from an opaque thread offset, so what a pass derives from them (keys, exp values,
// indices) is recomputed in that pass instead of being hoisted out of the searches' loops.
template <int NV>
struct RegRow {
  static constexpr bool kCacheable = NV <= 8;  // exp values kept too, up to 32768 tokens
  static constexpr int kSlots = NV * 8;
  uint4 r[NV];
  __device__ __forceinline__ void load(const uint16_t* row, int64_t V, bool vec) {
#pragma unroll
    for (int c = 0; c < NV; ++c)
      r[c] = load_chunk(row, V, vec, (static_cast<int64_t>(c) * kSampThreads + threadIdx.x) * 8);
  }
  template <typename G>
  __device__ __forceinline__ void chunks(G&& g) {
    const int32_t t8 = opaque_t8();
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      asm volatile("" : "+v"(r[c].x), "+v"(r[c].y), "+v"(r[c].z), "+v"(r[c].w));
      const uint32_t w[4] = {r[c].x, r[c].y, r[c].z, r[c].w};
      g(c, c * kSampThreads * 8 + t8, w);
    }
  }
};

// A row read again from global memory on every pass, for vocabularies beyond the registers' reach
// (the row stays in the caches between a workgroup's passes).
struct GlobalRow {
  static constexpr bool kCacheable = false;
  static constexpr int kSlots = 1;
  const uint16_t* p;
  int64_t V;
  bool vec;
  int n;
  __device__ __forceinline__ void load(const uint16_t* row, int64_t V_, bool vec_) {
    p = row, V = V_, vec = vec_;
    n = static_cast<int>((V + 8LL * kSampThreads - 1) / (8LL * kSampThreads));
  }
  template <typename G>
  __device__ __forceinline__ void chunks(G&& g) {
    const int32_t t8 = static_cast<int32_t>(threadIdx.x) * 8;
    for (int c = 0; c < n; ++c) {
      const int32_t base = c * kSampThreads * 8 + t8;
      const uint4 v = load_chunk(p, V, vec, base);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      g(0, base, w);
    }
  }
};

// The pass's accumulators, made opaque at the end of each chunk: the chunk's contributions are
// then added before the next chunk's words are read, instead of being sunk to the pass's end with
// every token's key kept live until there.
template <typename T>
__device__ __forceinline__ void fence1(T& v) {
  asm volatile("" : "+v"(v));
}
template <typename... T>
__device__ __forceinline__ void fence(T&... v) {
  (fence1(v), ...);
}

// f(slot, bf16 bits, token index) over the thread's tokens, in a fixed order; end() after each
// chunk (fences the pass's accumulators)
template <typename Row, typename F, typename G>
__device__ __forceinline__ void for_each(Row& row, F&& f, G&& end) {
  row.chunks([&](int c, int32_t base, const uint32_t (&w)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f(c * 8 + 2 * k, w[k] & 0xffffu, base + 2 * k);
      f(c * 8 + 2 * k + 1, w[k] >> 16, base + 2 * k + 1);
    }
    end();
  });
}

// One side's support and normaliser. Rows with a NaN or no finite maximum get kFlagNaN (the
// reference's softmax gives NaN there).
template <typename Row>
__device__ __forceinline__ SideStats compute_support(Row& r, int64_t V, const SideParams P, Red& red,
                                                     int& ph) {
  constexpr bool kCache = Row::kCacheable;
  SideStats st = {};
  float mx = -INFINITY;
  uint32_t bad = 0;
  for_each(r, [&](int, uint32_t h, int64_t) {
    bad |= (h & 0x7fffu) > 0x7f80u ? 1u : 0u;
    mx = fmaxf(mx, bf16f(h));
  }, [&] { fence(mx, bad); });
  const float m = block_max(mx, red, ph);
  const bool nan_row = block_count(bad, red, ph) > 0 || !(m > -INFINITY && m < INFINITY);
  st.m = m;
  st.rcp_t = P.temp ? P.rcp_t : 1.0f;
  st.flags = P.temp ? kFlagTemp : 0u;
  if (nan_row) {
    st.flags |= kFlagNaN;
    return st;
  }
  const RowCtx cx{m, st.rcp_t, P.temp != 0};
  float ec[kCache ? Row::kSlots : 1];
  if constexpr (kCache) for_each(r, [&](int s, uint32_t h, int64_t) { ec[s] = e_of(bf16f(h), cx); }, [] {});
  auto E = [&](int s, uint32_t h) -> float {
    if constexpr (kCache) return ec[s];
    else return e_of(bf16f(h), cx);
  };

  // top-p boundary (okey_p, n_p of c_p ties kept)
  bool have_p = false, have_k = false;
  uint32_t okey_p = 0, okey_k = 0;
  int64_t n_p = 0, c_p = 0, n_k = 0, c_k = 0;
  if (P.use_p) {
    double se = 0.0;
    for_each(r, [&](int s, uint32_t h, int64_t) { se += E(s, h); }, [&] { fence(se); });
    const double lim = static_cast<double>(P.top_p) * block_sum(se, red, ph);
    uint32_t lo = 0, hi = 0xffffu;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      double f = 0.0;
      for_each(r, [&](int s, uint32_t h, int64_t) { f += x_key(h) > mid ? E(s, h) : 0.0f; },
               [&] { fence(f); });
      if (block_sum(f, red, ph) <= lim) hi = mid;
      else lo = mid + 1;
    }
    if (lo != 0) {  // key 0 (a negative NaN) is never present: lo == 0 keeps every token
      have_p = true;
      const float xb = bf16f(x_bits_of_key(lo));
      okey_p = ord_key(ord_of(xb, cx));
      const float eb = e_of(xb, cx);
      double f = 0.0;
      uint32_t c = 0;
      for_each(r, [&](int s, uint32_t h, int64_t) {
        const uint32_t k = ord_key(ord_of(bf16f(h), cx));
        f += k > okey_p ? E(s, h) : 0.0f;
        c += k == okey_p ? 1u : 0u;
      }, [&] { fence(f, c); });
      const double above = block_sum(f, red, ph);
      c_p = block_count(c, red, ph);
      // the j-th tie (0-based, index order) has mass above + j * eb before it
      if (eb > 0.0f) {
        const double q = floor((lim - above) / static_cast<double>(eb));
        n_p = q + 1.0 >= static_cast<double>(c_p) ? c_p : static_cast<int64_t>(q) + 1;
      } else {
        n_p = c_p;
      }
    }
  }
  if (P.use_k) {  // 0 < top_k < V: the boundary is a present key
    have_k = true;
    uint32_t lo = 0, hi = 0xffffu;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      uint32_t cnt = 0;
      for_each(r, [&](int, uint32_t h, int64_t) { cnt += x_key(h) > mid ? 1u : 0u; },
               [&] { fence(cnt); });
      if (block_count(cnt, red, ph) <= P.top_k - 1) hi = mid;
      else lo = mid + 1;
    }
    okey_k = ord_key(ord_of(bf16f(x_bits_of_key(lo)), cx));
    uint32_t a = 0, c = 0;
    for_each(r, [&](int, uint32_t h, int64_t) {
      const uint32_t k = ord_key(ord_of(bf16f(h), cx));
      a += k > okey_k ? 1u : 0u;
      c += k == okey_k ? 1u : 0u;
    }, [&] { fence(a, c); });
    const int64_t above = block_count(a, red, ph);
    c_k = block_count(c, red, ph);
    n_k = P.top_k - above;
  }
  // both filters keep a prefix of the order: the shorter one wins
  uint32_t okey = 0;
  int64_t n = 0, cnt = 0;
  if (have_p && (!have_k || okey_p > okey_k)) {
    okey = okey_p, n = n_p, cnt = c_p;
  } else if (have_k && (!have_p || okey_k > okey_p)) {
    okey = okey_k, n = n_k, cnt = c_k;
  } else if (have_p && have_k) {
    okey = okey_p, n = n_p < n_k ? n_p : n_k, cnt = c_p;
  }
  st.okey = okey;
  st.last = 0x7fffffff;
  if (!have_p && !have_k) {
    st.flags |= kFlagAll;
  } else if (n < cnt) {
    // index of the n-th tie: the smallest j with n ties at indices <= j
    int64_t lo = 0, hi = V - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      uint32_t c = 0;
      for_each(r, [&](int, uint32_t h, int64_t idx) {
        c += ((idx <= mid) & (ord_key(ord_of(bf16f(h), cx)) == okey)) ? 1u : 0u;
      }, [&] { fence(c); });
      if (block_count(c, red, ph) >= n) hi = mid;
      else lo = mid + 1;
    }
    st.last = static_cast<int32_t>(lo);
  }
  double z = 0.0;
  uint32_t nm = 0;
  for_each(r, [&](int s, uint32_t h, int64_t idx) {
    const float x = bf16f(h);
    z += kept(st, ord_key(ord_of(x, cx)), idx) ? E(s, h) : 0.0f;
    nm += x == m ? 1u : 0u;
  }, [&] { fence(z, nm); });
  st.zinv = static_cast<float>(1.0 / block_sum(z, red, ph));
  st.nmax = static_cast<int32_t>(block_count(nm, red, ph));
  return st;
}

__device__ __forceinline__ void store_side(float* dst, const SideStats& s) {
  dst[0] = s.m;
  dst[1] = s.rcp_t;
  dst[2] = __uint_as_float(s.okey);
  dst[3] = __int_as_float(s.last);
  dst[4] = s.zinv;
  dst[5] = __uint_as_float(s.flags);
  dst[6] = __int_as_float(s.nmax);
  dst[7] = 0.0f;
}
__device__ __forceinline__ SideStats load_side(const float* src) {
  SideStats s;
  s.m = src[0];
  s.rcp_t = src[1];
  s.okey = __float_as_uint(src[2]);
  s.last = __float_as_int(src[3]);
  s.zinv = src[4];
  s.flags = __float_as_uint(src[5]);
  s.nmax = __float_as_int(src[6]);
  s.pad = 0;
  return s;
}

__device__ __forceinline__ bool row_vec(const uint16_t* p, int64_t V) {
  return V % 8 == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// ---- sampling_logits: the filtered fp32 logits and their gradient ------------------------------
template <typename Row>
__global__ void __launch_bounds__(kSampThreads) sampling_fwd_kernel(SampledArgs a) {
  __shared__ Red red;
  int ph = 0;
  const int64_t row = blockIdx.x, V = a.V;
  const SideParams px = a.px;
  Row r;
  r.load(a.x + row * V, V, row_vec(a.x, V));
  const SideStats s = compute_support(r, V, px, red, ph);
  const RowCtx cx = ctx_of(s);
  float* out = a.out + row * V;
  const bool nan_row = (s.flags & kFlagNaN) != 0;
  const bool vec_out = V % 4 == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0;
  r.chunks([&](int, int32_t base, const uint32_t (&w)[4]) {
    if (base >= V) return;
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = ord_of(bf16f(half_of(w, j)), cx);
      o[j] = nan_row ? __builtin_nanf("") : (kept(s, ord_key(v), base + j) ? v : -INFINITY);
    }
    if (vec_out && base + 8 <= V) {
      *reinterpret_cast<float4*>(out + base) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4*>(out + base + 4) = make_float4(o[4], o[5], o[6], o[7]);
    } else {
      for (int j = 0; j < 8 && base + j < V; ++j) out[base + j] = o[j];
    }
    __builtin_amdgcn_sched_barrier(0);
  });
  if (threadIdx.x == 0) store_side(a.stats + row * kSideWords, s);
}

// d logits = keep * g * (1/T), minus, with a temperature, sum(keep * g) / T shared by the tokens
// equal to the max (the gradient of the max subtraction; amax spreads it evenly over ties)
template <typename Row>
__global__ void __launch_bounds__(kSampThreads) sampling_bwd_kernel(SampledArgs a) {
  __shared__ Red red;
  int ph = 0;
  const int64_t row = blockIdx.x, V = a.V;
  Row r;
  r.load(a.x + row * V, V, row_vec(a.x, V));
  const SideStats s = load_side(a.stats + row * kSideWords);
  const RowCtx cx = ctx_of(s);
  const float* g = a.gout + row * V;
  uint16_t* dx = a.dx + row * V;
  const bool nan_row = (s.flags & kFlagNaN) != 0;
  const bool vec = V % 8 == 0 && (reinterpret_cast<uintptr_t>(a.gout) & 31) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.dx) & 15) == 0;
  // the chunk's eight upstream gradients (0 past the row's end)
  auto grads = [&](int32_t base, float (&gv)[8]) {
    if (vec && base + 8 <= V) {
      const float4 g0 = *reinterpret_cast<const float4*>(g + base);
      const float4 g1 = *reinterpret_cast<const float4*>(g + base + 4);
      gv[0] = g0.x, gv[1] = g0.y, gv[2] = g0.z, gv[3] = g0.w;
      gv[4] = g1.x, gv[5] = g1.y, gv[6] = g1.z, gv[7] = g1.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) gv[j] = base + j < V ? g[base + j] : 0.0f;
    }
  };
  float share = 0.0f;
  if ((s.flags & kFlagTemp) && !nan_row) {
    double sg = 0.0;
    r.chunks([&](int, int32_t base, const uint32_t (&w)[4]) {
      if (base >= V) return;
      float gv[8];
      grads(base, gv);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        sg += kept(s, ord_key(ord_of(bf16f(half_of(w, j)), cx)), base + j) ? gv[j] : 0.0f;
      fence(sg);
    });
    share = static_cast<float>(block_sum(sg, red, ph) * static_cast<double>(s.rcp_t) / s.nmax);
  }
  r.chunks([&](int, int32_t base, const uint32_t (&w)[4]) {
    if (base >= V) return;
    float gv[8];
    grads(base, gv);
    uint32_t packed[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float d[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float x = bf16f(half_of(w, 2 * k + h));
        float v = kept(s, ord_key(ord_of(x, cx)), base + 2 * k + h) ? gv[2 * k + h] * s.rcp_t : 0.0f;
        v -= x == s.m ? share : 0.0f;
        d[h] = nan_row ? __builtin_nanf("") : v;
      }
      packed[k] = pack_bf16x2(d[0], d[1]);
    }
    if (vec && base + 8 <= V) {
      *reinterpret_cast<uint4*>(dx + base) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    } else {
      for (int j = 0; j < 8 && base + j < V; ++j) dx[base + j] = static_cast<uint16_t>(half_of(packed, j));
    }
    __builtin_amdgcn_sched_barrier(0);
  });
}

// ---- sampled L1 ---------------------------------------------------------------------------------
template <typename Row>
__global__ void __launch_bounds__(kSampThreads) sampled_l1_fwd_kernel(SampledArgs a) {
  __shared__ Red red;
  int ph = 0;
  const int64_t row = blockIdx.x;
  int64_t yrow = row;
  if (a.yidx) {
    yrow = a.yidx[row];
    if (yrow < 0 || yrow >= a.trows) {  // the reference device-asserts; here a flag and a NaN row
      if (threadIdx.x == 0) {
        atomicOr(a.flags, 1);
        a.l1[row] = __builtin_nanf("");
        float* st = a.stats + row * kL1Words;
        for (int i = 0; i < kL1Words; ++i) st[i] = 0.0f;
        st[5] = __uint_as_float(kFlagNaN);
      }
      return;
    }
  }
  const int64_t V = a.V;
  const SideParams px = a.px, py = a.py;
  const uint16_t* xr = a.x + row * V;
  const uint16_t* yr = a.y + yrow * V;
  Row r;
  r.load(yr, V, row_vec(a.y, V));
  const SideStats sy = compute_support(r, V, py, red, ph);
  r.load(xr, V, row_vec(a.x, V));
  const SideStats sx = compute_support(r, V, px, red, ph);
  const bool nan_row = ((sx.flags | sy.flags) & kFlagNaN) != 0;
  double l1 = 0.0, pos = 0.0, neg = 0.0, zero = 0.0;
  if (!nan_row) {
    const bool yvec = row_vec(a.y, V);
    r.chunks([&](int, int32_t base, const uint32_t (&wx)[4]) {
      const uint4 yc = load_chunk(yr, V, yvec, base);
      const uint32_t wy[4] = {yc.x, yc.y, yc.z, yc.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = prob(sx, half_of(wx, j), base + j);
        const float q = prob(sy, half_of(wy, j), base + j);
        l1 += fabsf(p - q);
        pos += p > q ? p : 0.0f;
        neg += p < q ? p : 0.0f;
        zero += p == q ? p : 0.0f;
      }
      fence(l1, pos, neg, zero);
    });
  }
  const double t_l1 = block_sum(l1, red, ph);
  const double t_pos = block_sum(pos, red, ph);
  const double t_neg = block_sum(neg, red, ph);
  const double t_zero = block_sum(zero, red, ph);
  if (threadIdx.x == 0) {
    float* st = a.stats + row * kL1Words;
    store_side(st, sx);
    store_side(st + kSideWords, sy);
    st[16] = static_cast<float>(t_pos);
    st[17] = static_cast<float>(t_neg);
    st[18] = static_cast<float>(t_zero);
    for (int i = 19; i < kL1Words; ++i) st[i] = 0.0f;
    a.l1[row] = nan_row ? __builtin_nanf("") : static_cast<float>(t_l1);
  }
}

// d logits = g / T_draft * p * (sign(p - q) - sum p sign(p - q)), written per case without
// cancellation: 2 neg + zero (p > q), -(2 pos + zero) (p < q), neg - pos (p == q), where pos, neg
// and zero are the draft mass on tokens with p > q, p < q and p == q. Each workgroup takes one
// 2048-token segment of a row per loop step.
__global__ void __launch_bounds__(256) sampled_l1_bwd_kernel(SampledArgs a) {
  const int64_t segs = (a.V + 2047) / 2048;
  for (int64_t unit = blockIdx.x; unit < a.rows * segs; unit += gridDim.x) {
    const int64_t row = unit / segs;
    const int64_t base = (unit - row * segs) * 2048 + static_cast<int64_t>(threadIdx.x) * 8;
    const float* st = a.stats + row * kL1Words;
    const SideStats sx = load_side(st);
    const SideStats sy = load_side(st + kSideWords);
    const float pos = st[16], neg = st[17], zero = st[18];
    const float g = a.g_l1[row] * sx.rcp_t;
    const bool nan_row = ((sx.flags | sy.flags) & kFlagNaN) != 0;
    int64_t yrow = row;
    if (a.yidx) {
      yrow = a.yidx[row];
      if (yrow < 0 || yrow >= a.trows) yrow = 0;  // NaN row (flagged by the forward)
    }
    const uint16_t* xr = a.x + row * a.V;
    const uint16_t* yr = a.y + yrow * a.V;
    uint16_t* dr = a.dx + row * a.V;
    if (base >= a.V) continue;
    const float w_gt = g * (2.0f * neg + zero), w_lt = -g * (2.0f * pos + zero), w_eq = g * (neg - pos);
    for (int j = 0; j < 8 && base + j < a.V; ++j) {
      const int64_t idx = base + j;
      const float p = prob(sx, xr[idx], idx);
      const float q = prob(sy, yr[idx], idx);
      const float d = p * (p > q ? w_gt : (p < q ? w_lt : w_eq));
      dr[idx] = f32_to_bf16_bits(nan_row ? __builtin_nanf("") : d);
    }
  }
}

// ---- host side ----------------------------------------------------------------------------------
int side_params(double temperature, double top_p, int64_t top_k, int64_t V, SideParams* p) {
  if (!(temperature > 0.0) || !std::isfinite(temperature))
    return set_error(ASPEC_ERR_INVALID, "sampling temperature must be finite and > 0");
  if (!(top_p > 0.0 && top_p <= 1.0))
    return set_error(ASPEC_ERR_INVALID, "sampling top_p must lie in (0, 1]");
  if (top_k == 0 || top_k < -1)
    return set_error(ASPEC_ERR_INVALID, "sampling top_k must be -1 or >= 1");
  p->temp = temperature != 1.0;
  // the reference's (x - max) / T on CUDA multiplies by the fp32 reciprocal of T
  p->rcp_t = p->temp ? 1.0f / static_cast<float>(temperature) : 1.0f;
  p->top_p = static_cast<float>(top_p);
  p->use_p = top_p < 1.0;
  p->top_k = top_k;
  p->use_k = top_k > 0 && top_k < V;
  return ASPEC_OK;
}

// register chunks per thread for a vocabulary; 0: the row is read from global memory per pass
int chunks_for(int64_t V) {
  const int64_t per = (V + 8LL * kSampThreads - 1) / (8LL * kSampThreads);
  for (int nv : {1, 2, 4, 8, 16, 24})
    if (per <= nv) return nv;
  return 0;
}

#define ASPEC_SAMPLING_DISPATCH(KERNEL, NV, ...)                                                    \
  switch (NV) {                                                                                     \
    case 1: hipLaunchKernelGGL(KERNEL<RegRow<1>>, __VA_ARGS__); break;                               \
    case 2: hipLaunchKernelGGL(KERNEL<RegRow<2>>, __VA_ARGS__); break;                               \
    case 4: hipLaunchKernelGGL(KERNEL<RegRow<4>>, __VA_ARGS__); break;                               \
    case 8: hipLaunchKernelGGL(KERNEL<RegRow<8>>, __VA_ARGS__); break;                               \
    case 16: hipLaunchKernelGGL(KERNEL<RegRow<16>>, __VA_ARGS__); break;                             \
    case 24: hipLaunchKernelGGL(KERNEL<RegRow<24>>, __VA_ARGS__); break;                             \
    default: hipLaunchKernelGGL(KERNEL<GlobalRow>, __VA_ARGS__); break;                              \
  }

int check_rows(int64_t rows, int64_t V, const void* x) {
  if (rows <= 0 || V <= 0 || !x) return set_error(ASPEC_ERR_INVALID, "sampling needs nonempty bf16 logits");
  if (rows > 0x7fffffffLL) return set_error(ASPEC_ERR_UNSUPPORTED, "sampling takes at most 2^31 - 1 rows");
  if (V > (1LL << 24))
    return set_error(ASPEC_ERR_UNSUPPORTED, "sampling covers vocabularies up to 2^24 tokens");
  return ASPEC_OK;
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_sampling_stats_floats(void) { return kSideWords; }
extern "C" int aspec_sampled_l1_stats_floats(void) { return kL1Words; }

extern "C" int aspec_sampling_logits_fwd(const void* logits, int64_t rows, int64_t vocab,
                                         double temperature, double top_p, int64_t top_k, float* out,
                                         float* stats, void* stream) {
  int rc = check_rows(rows, vocab, logits);
  if (rc) return rc;
  if (!out || !stats) return set_error(ASPEC_ERR_INVALID, "sampling needs output and stats buffers");
  SampledArgs a = {};
  a.x = static_cast<const uint16_t*>(logits);
  a.rows = rows;
  a.V = vocab;
  a.out = out;
  a.stats = stats;
  if ((rc = side_params(temperature, top_p, top_k, vocab, &a.px))) return rc;
  ASPEC_SAMPLING_DISPATCH(sampling_fwd_kernel, chunks_for(vocab), dim3(static_cast<uint32_t>(rows)),
                          dim3(kSampThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("sampling logits");
}

extern "C" int aspec_sampling_logits_bwd(const void* logits, const float* grad_out, const float* stats,
                                         int64_t rows, int64_t vocab, void* grad_logits, void* stream) {
  int rc = check_rows(rows, vocab, logits);
  if (rc) return rc;
  if (!grad_out || !stats || !grad_logits)
    return set_error(ASPEC_ERR_INVALID, "sampling backward needs gradient, stats and output buffers");
  SampledArgs a = {};
  a.x = static_cast<const uint16_t*>(logits);
  a.rows = rows;
  a.V = vocab;
  a.gout = grad_out;
  a.stats = const_cast<float*>(stats);
  a.dx = static_cast<uint16_t*>(grad_logits);
  ASPEC_SAMPLING_DISPATCH(sampling_bwd_kernel, chunks_for(vocab), dim3(static_cast<uint32_t>(rows)),
                          dim3(kSampThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("sampling logits backward");
}

extern "C" int aspec_sampled_l1_fwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                                    int64_t teacher_rows, int64_t rows, int64_t vocab,
                                    double draft_temperature, double draft_top_p, int64_t draft_top_k,
                                    double target_temperature, double target_top_p, int64_t target_top_k,
                                    float* l1_out, float* stats, int32_t* status_flags, void* stream) {
  int rc = check_rows(rows, vocab, logits);
  if (rc) return rc;
  if (!teacher || !l1_out || !stats || !status_flags)
    return set_error(ASPEC_ERR_INVALID, "sampled L1 needs teacher logits, output, stats and status buffers");
  if (teacher_index && teacher_rows <= 0) return set_error(ASPEC_ERR_INVALID, "indexed teacher table is empty");
  SampledArgs a = {};
  a.x = static_cast<const uint16_t*>(logits);
  a.y = static_cast<const uint16_t*>(teacher);
  a.yidx = teacher_index;
  a.trows = teacher_index ? teacher_rows : rows;
  a.rows = rows;
  a.V = vocab;
  a.l1 = l1_out;
  a.stats = stats;
  a.flags = status_flags;
  if ((rc = side_params(draft_temperature, draft_top_p, draft_top_k, vocab, &a.px))) return rc;
  if ((rc = side_params(target_temperature, target_top_p, target_top_k, vocab, &a.py))) return rc;
  ASPEC_SAMPLING_DISPATCH(sampled_l1_fwd_kernel, chunks_for(vocab), dim3(static_cast<uint32_t>(rows)),
                          dim3(kSampThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("sampled L1 forward");
}

extern "C" int aspec_sampled_l1_bwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                                    int64_t teacher_rows, int64_t rows, int64_t vocab, const float* stats,
                                    const float* grad_l1, void* grad_logits, void* stream) {
  int rc = check_rows(rows, vocab, logits);
  if (rc) return rc;
  if (!teacher || !stats || !grad_l1 || !grad_logits)
    return set_error(ASPEC_ERR_INVALID, "sampled L1 backward needs teacher logits, stats, gradients and output");
  SampledArgs a = {};
  a.x = static_cast<const uint16_t*>(logits);
  a.y = static_cast<const uint16_t*>(teacher);
  a.yidx = teacher_index;
  a.trows = teacher_index ? teacher_rows : rows;
  a.rows = rows;
  a.V = vocab;
  a.stats = const_cast<float*>(stats);
  a.g_l1 = grad_l1;
  a.dx = static_cast<uint16_t*>(grad_logits);
  const int64_t units = rows * ((vocab + 2047) / 2048);
  const int64_t grid = units < 256 * 64 ? units : 256 * 64;
  hipLaunchKernelGGL(sampled_l1_bwd_kernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("sampled L1 backward");
}
