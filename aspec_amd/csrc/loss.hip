// Vocabulary-sliced loss kernels: softmax-L1 (tiled_l1.py semantics) and cross-entropy, forward
// and backward, alone or fused. HBM-bound streaming reductions.
//
// Forward, one workgroup per row:
//   resident path (V % 8 == 0, V <= 1024*8*4): 1024 threads read the draft row and the teacher row
//   from HBM exactly once into registers, then reduce max / sum / |p - q| / sign masses;
//   streaming path (any V): 256 threads, element loads, the rows re-read from cache per pass.
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

// Emits nothing; makes the packed chunks look modified, so each pass unpacks them afresh instead
// of the compiler keeping 16 unpacked floats per chunk alive across passes (which spills).
template <int NV>
__device__ __forceinline__ void opaque_chunks(uint4 (&v)[NV]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) asm volatile("" : "+v"(v[j].x), "+v"(v[j].y), "+v"(v[j].z), "+v"(v[j].w));
}
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// This thread's (max, sum-exp) over the packed row chunks `v`.
template <int NV>
__device__ __forceinline__ void thread_max_sum(uint4 (&v)[NV], float& m, float& s) {
  m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) m = fmaxf(m, fmaxf(lo_bf(w[e]), hi_bf(w[e])));
  }
  opaque_chunks(v);
  const float nm = m == -INFINITY ? 0.f : neg_scaled_max(m);
  s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) s += scaled_exp2(lo_bf(w[e]), nm) + scaled_exp2(hi_bf(w[e]), nm);
    __builtin_amdgcn_sched_barrier(0);  // one chunk at a time: keeps the exps from piling up in registers
  }
}

// Row-resident forward: 1024 threads hold one row of draft and teacher logits as packed bf16
// (8*NV registers per tensor), read from HBM exactly once. At <= 64 VGPRs two rows share a CU, so
// one row's loads overlap the other's arithmetic. Each thread reduces its own chunk to a
// (max, sum-exp) pair; one block merge gives the row's softmax, a second pass the L1 terms.
template <int NV>
__global__ void __launch_bounds__(1024, 8) loss_fwd_resident(LossArgs a) {
  __shared__ float scratch[4 * 32];
  const int64_t row = blockIdx.x;
  const bool has_y = a.y != nullptr;
  const int64_t trow = has_y ? teacher_row(a, row) : 0;
  const uint16_t* xr = a.x + row * a.V;
  const uint16_t* yr = has_y && trow >= 0 ? a.y + trow * a.V : nullptr;
  uint4 xs[NV], ys[NV];
  const uint4* xq = reinterpret_cast<const uint4*>(xr);
  const uint4* yq = reinterpret_cast<const uint4*>(yr);
  const uint32_t nchunks = static_cast<uint32_t>(a.V / 8);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t chunk = j * 1024u + threadIdx.x;  // 32-bit offsets: one base register pair
    xs[j] = make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u);  // -inf padding
    ys[j] = xs[j];
    if (chunk < nchunks) {
      xs[j] = xq[chunk];
      if (yr) ys[j] = yq[chunk];
    }
  }
  float m[2], s[2];
  thread_max_sum(xs, m[0], s[0]);
  thread_max_sum(ys, m[1], s[1]);
  opaque_chunks(xs);
  opaque_chunks(ys);
  block_max_sum<2>(m, s, scratch);
  const float nmx = neg_scaled_max(m[0]), nmy = neg_scaled_max(m[1]);
  const float ix = 1.f / s[0], iy = 1.f / s[1];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (has_y) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const uint32_t xw[4] = {xs[j].x, xs[j].y, xs[j].z, xs[j].w};
      const uint32_t yw[4] = {ys[j].x, ys[j].y, ys[j].z, ys[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        l1_terms(scaled_exp2(lo_bf(xw[e]), nmx) * ix, scaled_exp2(lo_bf(yw[e]), nmy) * iy, acc[0], acc[1], acc[2], acc[3]);
        l1_terms(scaled_exp2(hi_bf(xw[e]), nmx) * ix, scaled_exp2(hi_bf(yw[e]), nmy) * iy, acc[0], acc[1], acc[2], acc[3]);
      }
      __builtin_amdgcn_sched_barrier(0);
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

int launch_fwd(const LossArgs& a, hipStream_t s) {
  const bool vec = a.V % 8 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                   (!a.y || (reinterpret_cast<uintptr_t>(a.y) & 15) == 0);
  const dim3 grid(static_cast<uint32_t>(a.rows));
  if (vec && a.V <= 1024 * 8 * 1) {
    hipLaunchKernelGGL(loss_fwd_resident<1>, grid, dim3(1024), 0, s, a);
  } else if (vec && a.V <= 1024 * 8 * 2) {
    hipLaunchKernelGGL(loss_fwd_resident<2>, grid, dim3(1024), 0, s, a);
  } else if (vec && a.V <= 1024 * 8 * 4) {
    hipLaunchKernelGGL(loss_fwd_resident<4>, grid, dim3(1024), 0, s, a);
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
    hipLaunchKernelGGL(loss_bwd_kernel<true>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(loss_bwd_kernel<false>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, a);
  }
  return check_launch("loss backward");
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

extern "C" int aspec_ce_l1_fwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                               int64_t teacher_rows, const int64_t* targets, int64_t ignore_index,
                               int64_t rows, int64_t vocab, float* l1_out, float* ce_out,
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
  return launch_fwd(a, static_cast<hipStream_t>(stream));
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
