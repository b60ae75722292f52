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

template <int NV>
__global__ void __launch_bounds__(1024) loss_fwd_resident(LossArgs a) {
  __shared__ float scratch[4 * 32];
  const int64_t row = blockIdx.x;
  const bool has_y = a.y != nullptr;
  const int64_t trow = has_y ? teacher_row(a, row) : 0;
  const uint16_t* xr = a.x + row * a.V;
  const uint16_t* yr = has_y && trow >= 0 ? a.y + trow * a.V : nullptr;
  constexpr int E = NV * 8;
  float xv[E], yv[E];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t col = (static_cast<int64_t>(j) * blockDim.x + threadIdx.x) * 8;
    uint4 xs = make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u);  // -inf padding
    uint4 ys = xs;
    if (col < a.V) {
      xs = *reinterpret_cast<const uint4*>(xr + col);
      if (yr) ys = *reinterpret_cast<const uint4*>(yr + col);
    }
    const uint32_t xw[4] = {xs.x, xs.y, xs.z, xs.w};
    const uint32_t yw[4] = {ys.x, ys.y, ys.z, ys.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[j * 8 + 2 * e] = __uint_as_float(xw[e] << 16);
      xv[j * 8 + 2 * e + 1] = __uint_as_float(xw[e] & 0xffff0000u);
      yv[j * 8 + 2 * e] = __uint_as_float(yw[e] << 16);
      yv[j * 8 + 2 * e + 1] = __uint_as_float(yw[e] & 0xffff0000u);
    }
  }
  float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
  for (int i = 0; i < E; ++i) {
    mx[0] = fmaxf(mx[0], xv[i]);
    mx[1] = fmaxf(mx[1], yv[i]);
  }
  block_reduce<2, true>(mx, scratch);
  float sums[2] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < E; ++i) {
    xv[i] = fexp2((xv[i] - mx[0]) * kLog2e);
    yv[i] = fexp2((yv[i] - mx[1]) * kLog2e);
    sums[0] += xv[i];
    sums[1] += yv[i];
  }
  block_reduce<2, false>(sums, scratch);
  const float ix = 1.f / sums[0], iy = 1.f / sums[1];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (has_y) {
#pragma unroll
    for (int i = 0; i < E; ++i) l1_terms(xv[i] * ix, yv[i] * iy, acc[0], acc[1], acc[2], acc[3]);
    block_reduce<4, false>(acc, scratch);
  }
  if (threadIdx.x == 0) {
    const float lse = logf(sums[0]) + mx[0];
    float* st = a.stats + row * kStats;
    st[0] = mx[0]; st[1] = ix; st[2] = mx[1]; st[3] = iy;
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
  float mx[2] = {-INFINITY, -INFINITY};
  for (int64_t i = threadIdx.x; i < a.V; i += blockDim.x) {
    mx[0] = fmaxf(mx[0], bf(xr[i]));
    if (yr) mx[1] = fmaxf(mx[1], bf(yr[i]));
  }
  block_reduce<2, true>(mx, scratch);
  float sums[2] = {0.f, 0.f};
  for (int64_t i = threadIdx.x; i < a.V; i += blockDim.x) {
    sums[0] += fexp2((bf(xr[i]) - mx[0]) * kLog2e);
    if (yr) sums[1] += fexp2((bf(yr[i]) - mx[1]) * kLog2e);
  }
  block_reduce<2, false>(sums, scratch);
  const float ix = 1.f / sums[0], iy = 1.f / sums[1];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (has_y) {
    for (int64_t i = threadIdx.x; i < a.V; i += blockDim.x) {
      const float p = fexp2((bf(xr[i]) - mx[0]) * kLog2e) * ix;
      const float q = yr ? fexp2((bf(yr[i]) - mx[1]) * kLog2e) * iy : NAN;
      l1_terms(p, q, acc[0], acc[1], acc[2], acc[3]);
    }
    block_reduce<4, false>(acc, scratch);
  }
  if (threadIdx.x == 0) {
    const float lse = logf(sums[0]) + mx[0];
    float* st = a.stats + row * kStats;
    st[0] = mx[0]; st[1] = ix; st[2] = mx[1]; st[3] = iy;
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
  const float p = fexp2((x - st[0]) * kLog2e) * st[1];
  float d = 0.f;
  if (has_y) {
    const float q = fexp2((y - st[2]) * kLog2e) * st[3];
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
