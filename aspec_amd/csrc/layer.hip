// The rest of one DSpark draft layer's training step (aspec/models/draft/dflash.py:968-1062,
// 1258-1284, 1470-1472) and its optimizer (aspec/training/optimizer.py:40-164): RMSNorm with an
// optional fused residual add, the SwiGLU activation, and a one-pass AdamW over flat fp32
// master weights. All are HBM-bound.
//
// RMSNorm (`_dflash_rms_norm`, dflash.py:282-293, and the fused rmsnorm the reference runs on the
// GPU, dflash.py:181-188): y = x (+ residual, rounded to bf16 as the reference's residual add
// is), rstd = 1/sqrt(mean(y^2) + eps), out = bf16(y * rstd * w) with one rounding. One wave per
// row (hidden a multiple of 8, at most 8192): lane l holds 8-element chunks l, l + 64, ...
// Backward with g = dout * w and n = y * rstd: dy = rstd * (g - n * mean(g * n)) + dy_extra
// (the gradient reaching y directly, for the residual add); dw = sum over rows of dout * n in
// fp32, per-wave partials reduced in a fixed order (deterministic).
//
// SwiGLU (`DFlashMLP.forward`, dflash.py:967-980): gate and up come from one GEMM as
// gu = [gate | up] (rows x 2F); out = silu(gate) * up in fp32, one bf16 rounding. Backward:
// dgate = dout * up * s * (1 + gate * (1 - s)), dup = dout * gate * s, s = sigmoid(gate).
//
// AdamW (`BF16Optimizer.step` with torch's fused AdamW): every trainable bf16 parameter is a
// view of one flat bf16 buffer with an fp32 master copy and fp32 moments; gradients land in one
// flat bf16 buffer. Step: ||g|| over the flat gradients (fp32 partials, fp64 final sum), clip
// coefficient min(max_norm / (||g|| + 1e-6), 1), skip everything (step count included) when
// ||g|| is not finite, else p *= 1 - lr*wd; m = lerp(m, g, 1 - b1); v = b2 v + (1 - b2) g^2;
// p -= lr / (1 - b1^t) * m / (sqrt(v) / sqrt(1 - b2^t) + eps), and the bf16 parameter is the
// round-to-nearest-even copy of p. The step count lives on the device, so no host sync.
#include <math.h>

#include <algorithm>

#include "common.h"

namespace aspec {
namespace {

constexpr int kNormMaxChunks = 16;  // hidden <= 16 * 64 * 8 = 8192
constexpr int kNormWaves = 4;       // rows (waves) per 256-thread workgroup
constexpr int kNormBwdGroups = 1024;  // backward grid, one partial dw row each (fixed: deterministic dw)

__device__ __forceinline__ void unpack8(const uint4& v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

struct NormArgs {
  const uint16_t* x;
  const uint16_t* residual;
  const uint16_t* w;
  uint16_t* y;      // x + residual (forward, when residual)
  uint16_t* out;    // forward output
  float* rstd;      // [rows]
  const uint16_t* dout;
  const uint16_t* dy_extra;
  const uint16_t* y_in;  // backward: the normalized input
  uint16_t* dy;
  float* partials;  // [kNormBwdGroups][hidden]
  float* dw;
  int64_t rows;
  int hidden;
  float eps;
};

__global__ void __launch_bounds__(64 * kNormWaves) rmsnorm_fwd_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int nch = a.hidden >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(a.x + row * a.hidden);
  const uint4* rr = a.residual ? reinterpret_cast<const uint4*>(a.residual + row * a.hidden) : nullptr;
  uint4 yv[kNormMaxChunks];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormMaxChunks; ++c) {
    const int ch = c * 64 + lane;
    if (ch >= nch) break;
    uint4 v = xr[ch];
    if (rr) {  // the residual add rounds to bf16, as the reference's bf16 add does
      float f[8], g[8];
      unpack8(v, f);
      unpack8(rr[ch], g);
#pragma unroll
      for (int k = 0; k < 8; ++k) f[k] += g[k];
      v = pack8(f);
      reinterpret_cast<uint4*>(a.y + row * a.hidden)[ch] = v;
    }
    yv[c] = v;
    float f[8];
    unpack8(v, f);
#pragma unroll
    for (int k = 0; k < 8; ++k) ss = fmaf(f[k], f[k], ss);
  }
  ss = wave_sum(ss);
  const float rstd = 1.f / sqrtf(ss / static_cast<float>(a.hidden) + a.eps);
  const uint4* wr = reinterpret_cast<const uint4*>(a.w);
  uint4* orow = reinterpret_cast<uint4*>(a.out + row * a.hidden);
#pragma unroll
  for (int c = 0; c < kNormMaxChunks; ++c) {
    const int ch = c * 64 + lane;
    if (ch >= nch) break;
    float f[8], w[8];
    unpack8(yv[c], f);
    unpack8(wr[ch], w);
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = f[k] * rstd * w[k];
    orow[ch] = pack8(f);
  }
  if (lane == 0) a.rstd[row] = rstd;
}

// One 256-thread workgroup per row (thread t holds chunks t, t + 256, ...: kNormBwdChunks of them,
// 2 for hidden 4096, at most 4), rows strided over the fixed grid; each thread accumulates dw for
// its columns, written as one partial row per workgroup.
constexpr int kNormBwdThreads = 256;

template <int kNormBwdChunks>
__global__ void __launch_bounds__(kNormBwdThreads) rmsnorm_bwd_kernel(NormArgs a) {
  __shared__ float red[kNormBwdThreads / 64];
  const int tid = threadIdx.x;
  const int nch = a.hidden >> 3;
  const uint4* wr = reinterpret_cast<const uint4*>(a.w);
  float dwacc[kNormBwdChunks][8];
  float w[kNormBwdChunks][8];
#pragma unroll
  for (int c = 0; c < kNormBwdChunks; ++c) {
    const int ch = c * kNormBwdThreads + tid;
    const uint4 wv = ch < nch ? wr[ch] : make_uint4(0, 0, 0, 0);
    unpack8(wv, w[c]);
#pragma unroll
    for (int k = 0; k < 8; ++k) dwacc[c][k] = 0.f;
  }
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const uint4* gr = reinterpret_cast<const uint4*>(a.dout + row * a.hidden);
    const uint4* yr = reinterpret_cast<const uint4*>(a.y_in + row * a.hidden);
    const float rstd = a.rstd[row];
    float g[kNormBwdChunks][8], n[kNormBwdChunks][8];
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < kNormBwdChunks; ++c) {
      const int ch = c * kNormBwdThreads + tid;
      const bool in = ch < nch;
      unpack8(in ? gr[ch] : make_uint4(0, 0, 0, 0), g[c]);
      unpack8(in ? yr[ch] : make_uint4(0, 0, 0, 0), n[c]);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        n[c][k] *= rstd;
        dot = fmaf(g[c][k] * w[c][k], n[c][k], dot);
        dwacc[c][k] = fmaf(g[c][k], n[c][k], dwacc[c][k]);
      }
    }
    dot = wave_sum(dot);
    if ((tid & 63) == 0) red[tid >> 6] = dot;
    __syncthreads();
    dot = ((red[0] + red[1]) + (red[2] + red[3])) / static_cast<float>(a.hidden);
    __syncthreads();  // red is rewritten by the next row
    uint4* dyr = reinterpret_cast<uint4*>(a.dy + row * a.hidden);
    const uint4* er = a.dy_extra ? reinterpret_cast<const uint4*>(a.dy_extra + row * a.hidden) : nullptr;
#pragma unroll
    for (int c = 0; c < kNormBwdChunks; ++c) {
      const int ch = c * kNormBwdThreads + tid;
      if (ch < nch) {
        float d[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) d[k] = rstd * (g[c][k] * w[c][k] - n[c][k] * dot);
        if (er) {
          float e[8];
          unpack8(er[ch], e);
#pragma unroll
          for (int k = 0; k < 8; ++k) d[k] += e[k];
        }
        dyr[ch] = pack8(d);
      }
    }
  }
  float* part = a.partials + static_cast<int64_t>(blockIdx.x) * a.hidden;
#pragma unroll
  for (int c = 0; c < kNormBwdChunks; ++c) {
    const int ch = c * kNormBwdThreads + tid;
    if (ch < nch) {
      reinterpret_cast<f32x4*>(part + ch * 8)[0] = f32x4{dwacc[c][0], dwacc[c][1], dwacc[c][2], dwacc[c][3]};
      reinterpret_cast<f32x4*>(part + ch * 8)[1] = f32x4{dwacc[c][4], dwacc[c][5], dwacc[c][6], dwacc[c][7]};
    }
  }
}

// dw[col] = sum of the partial rows, in a fixed order: a 1024-thread workgroup owns 64 columns
// (lane = column); wave w sums rows w, w + 16, ... and the 16 wave sums are added in wave order.
constexpr int kColWaves = 16;

__global__ void __launch_bounds__(64 * kColWaves) column_sum_kernel(const float* partials, int nparts,
                                                                   int cols, float* out) {
  __shared__ float part[kColWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (col < cols)
    for (int p = wave; p < nparts; p += kColWaves) s += partials[static_cast<int64_t>(p) * cols + col];
  part[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && col < cols) {
    float t = part[0][lane];
#pragma unroll
    for (int w = 1; w < kColWaves; ++w) t += part[w][lane];
    out[col] = t;
  }
}

struct SwiGluArgs {
  const uint16_t* gu;
  const uint16_t* dout;
  uint16_t* out;
  uint16_t* dgu;
  int64_t rows;
  int64_t ffn;  // F (gu rows hold 2F)
};

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }

__global__ void __launch_bounds__(256) swiglu_fwd_kernel(SwiGluArgs a) {
  const int64_t per_row = a.ffn >> 3;
  const int64_t total = a.rows * per_row;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = t / per_row, c = t - row * per_row;
    const uint4* base = reinterpret_cast<const uint4*>(a.gu + row * 2 * a.ffn);
    float g[8], u[8], o[8];
    unpack8(base[c], g);
    unpack8(base[per_row + c], u);
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = g[k] * sigmoidf(g[k]) * u[k];
    reinterpret_cast<uint4*>(a.out + row * a.ffn)[c] = pack8(o);
  }
}

__global__ void __launch_bounds__(256) swiglu_bwd_kernel(SwiGluArgs a) {
  const int64_t per_row = a.ffn >> 3;
  const int64_t total = a.rows * per_row;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = t / per_row, c = t - row * per_row;
    const uint4* base = reinterpret_cast<const uint4*>(a.gu + row * 2 * a.ffn);
    float g[8], u[8], d[8], dg[8], du[8];
    unpack8(base[c], g);
    unpack8(base[per_row + c], u);
    unpack8(reinterpret_cast<const uint4*>(a.dout + row * a.ffn)[c], d);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float s = sigmoidf(g[k]);
      du[k] = d[k] * g[k] * s;
      dg[k] = d[k] * u[k] * s * (1.f + g[k] * (1.f - s));
    }
    uint4* drow = reinterpret_cast<uint4*>(a.dgu + row * 2 * a.ffn);
    drow[c] = pack8(dg);
    drow[per_row + c] = pack8(du);
  }
}

// ---------------------------------------------------------------------------------------------
// AdamW
// ---------------------------------------------------------------------------------------------
constexpr int kAdamBlocks = 1024;  // norm partials (fixed: deterministic norm)

constexpr int kMaxGradSegments = 64;

// Device-side optimizer state: written by the finalize kernel, read by the update kernel. Each
// gradient segment (one parameter, or the whole flat buffer) keeps its own step count, as torch's
// AdamW keeps one per parameter: a parameter without a gradient in some steps takes its bias
// corrections from the steps in which it had one.
struct AdamState {
  int64_t step;      // completed steps (non-finite steps excluded)
  float coef;        // clip coefficient applied to the gradients
  int32_t skip;      // non-finite gradient norm: this step changes nothing
  float bc1, bc2s;   // segment 0's 1 - b1^t and sqrt(1 - b2^t) of the step being taken
  float norm;        // gradient norm before clipping
  float pad[2];
  int64_t seg_step[kMaxGradSegments];  // steps in which segment s had a gradient
  float seg_bc1[kMaxGradSegments];     // 1 - b1^t_s of the step being taken
  float seg_bc2s[kMaxGradSegments];    // sqrt(1 - b2^t_s)
};
static_assert(offsetof(AdamState, norm) == 24 && offsetof(AdamState, seg_step) == 40 &&
                  sizeof(AdamState) == 40 + 16 * kMaxGradSegments,
              "AdamState layout is part of the C ABI");

// Where the gradients are: one flat buffer (one segment) or one tensor per parameter, in the
// parameters' flat order. Segment s covers flat elements [end[s-1], end[s]); ptr[s] is its bf16
// gradient, or null for a parameter without one (it contributes nothing to the norm and is not
// updated, as torch's optimizers skip a parameter whose grad is None); bit s of `active` is set
// iff ptr[s] is not null. Every segment but the last holds a multiple of 8 elements and starts
// 16-byte aligned, so an 8-element chunk never straddles two segments.
struct GradTable {
  int nseg;
  uint64_t active;
  int64_t end[kMaxGradSegments];
  const uint16_t* ptr[kMaxGradSegments];
};

// The gradient of flat element e (null: none) and its segment, by a uniform scan of the table (a
// handful of scalar loads and lane selects per 8-element chunk).
__device__ __forceinline__ const uint16_t* grad_at(const GradTable& t, int64_t e, int& seg) {
  const uint16_t* p = nullptr;
  int64_t start = 0;
  seg = 0;
  for (int s = 0; s < t.nseg; ++s) {
    const int64_t end = t.end[s];
    if (e >= start && e < end) {
      p = t.ptr[s] ? t.ptr[s] + (e - start) : nullptr;
      seg = s;
    }
    start = end;
  }
  return p;
}

__global__ void __launch_bounds__(256) grad_sumsq_kernel(GradTable g, int64_t n, float* partials) {
  __shared__ float red[4];
  float s = 0.f;
  const int64_t n8 = n >> 3;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int seg;
    const uint16_t* gp = grad_at(g, i << 3, seg);
    if (!gp) continue;
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(gp), f);
#pragma unroll
    for (int k = 0; k < 8; ++k) s = fmaf(f[k], f[k], s);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    int seg;
    const uint16_t* gp = grad_at(g, (n8 << 3) + threadIdx.x, seg);
    if (gp) {
      const float f = bf16_to_f32(*gp);
      s = fmaf(f, f, s);
    }
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ void __launch_bounds__(64) adam_finalize_kernel(const float* partials, int nparts,
                                                           float max_norm, float b1, float b2,
                                                           int nseg, uint64_t active,
                                                           AdamState* st) {
  // fixed-order fp64 sum of the partials (one wave, lane-strided then a tree)
  double s = 0.0;
  for (int i = threadIdx.x; i < nparts; i += 64) s += static_cast<double>(partials[i]);
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  const float norm = static_cast<float>(sqrt(s));
  const bool finite = isfinite(norm);
  // lane j: segment j's step count and bias corrections
  const int j = threadIdx.x;
  if (j < nseg) {
    const int64_t t = st->seg_step[j] + ((finite && ((active >> j) & 1)) ? 1 : 0);
    st->seg_step[j] = t;
    st->seg_bc1[j] = static_cast<float>(1.0 - pow(static_cast<double>(b1), static_cast<double>(t)));
    st->seg_bc2s[j] = static_cast<float>(sqrt(1.0 - pow(static_cast<double>(b2), static_cast<double>(t))));
    if (j == 0) {
      st->bc1 = st->seg_bc1[0];
      st->bc2s = st->seg_bc2s[0];
    }
  }
  if (j == 0) {
    st->norm = norm;
    st->skip = finite ? 0 : 1;
    float coef = 1.f;
    if (max_norm > 0.f) coef = fminf(max_norm / (norm + 1e-6f), 1.f);
    st->coef = coef;
    st->step += finite ? 1 : 0;
  }
}

struct AdamArgs {
  uint16_t* param;
  float* master;
  float* m;
  float* v;
  GradTable grad;
  int64_t n;
  float lr, wd, b1, b2, eps;
  const AdamState* st;
};

__device__ __forceinline__ float adam_one(float g, float& p, float& m, float& v, const AdamArgs& a,
                                          float step_size, float decay, float bc2s) {
  p *= decay;
  m = m + (1.f - a.b1) * (g - m);  // lerp(m, g, 1 - b1)
  v = a.b2 * v + (1.f - a.b2) * g * g;
  p = p - step_size * (m / (sqrtf(v) / bc2s + a.eps));
  return p;
}

// Eight parameters per thread and iteration (16-byte bf16, 2 x 16-byte fp32 accesses), scalar tail.
__global__ void __launch_bounds__(256) adam_update_kernel(AdamArgs a) {
  const float coef = a.st->coef;
  if (a.st->skip) return;
  const float decay = 1.f - a.lr * a.wd;
  const int64_t n8 = a.n >> 3;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8; i += stride) {
    int seg;
    const uint16_t* gp = grad_at(a.grad, i << 3, seg);
    if (!gp) continue;
    const float step_size = a.lr / a.st->seg_bc1[seg];
    const float bc2s = a.st->seg_bc2s[seg];
    float g[8];
    unpack8(*reinterpret_cast<const uint4*>(gp), g);
    f32x4* mp = reinterpret_cast<f32x4*>(a.master) + 2 * i;
    f32x4* mm = reinterpret_cast<f32x4*>(a.m) + 2 * i;
    f32x4* mv = reinterpret_cast<f32x4*>(a.v) + 2 * i;
    const f32x4 p4[2] = {mp[0], mp[1]}, m4[2] = {mm[0], mm[1]}, v4[2] = {mv[0], mv[1]};
    float p[8], m[8], v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      p[k] = p4[k >> 2][k & 3];
      m[k] = m4[k >> 2][k & 3];
      v[k] = v4[k >> 2][k & 3];
      adam_one(g[k] * coef, p[k], m[k], v[k], a, step_size, decay, bc2s);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      mp[h] = f32x4{p[4 * h], p[4 * h + 1], p[4 * h + 2], p[4 * h + 3]};
      mm[h] = f32x4{m[4 * h], m[4 * h + 1], m[4 * h + 2], m[4 * h + 3]};
      mv[h] = f32x4{v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
    }
    reinterpret_cast<uint4*>(a.param)[i] = pack8(p);
  }
  for (int64_t i = (n8 << 3) + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    int seg;
    const uint16_t* gp = grad_at(a.grad, i, seg);
    if (!gp) continue;
    const float step_size = a.lr / a.st->seg_bc1[seg];
    float p = a.master[i], m = a.m[i], v = a.v[i];
    adam_one(bf16_to_f32(*gp) * coef, p, m, v, a, step_size, decay, a.st->seg_bc2s[seg]);
    a.master[i] = p;
    a.m[i] = m;
    a.v[i] = v;
    a.param[i] = f32_to_bf16_bits(p);
  }
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_rmsnorm_fwd(const void* x, const void* residual, const void* weight, int64_t rows,
                                 int64_t hidden, float eps, void* y_out, void* out, float* rstd,
                                 void* stream) {
  if (rows <= 0 || hidden <= 0) return set_error(ASPEC_ERR_INVALID, "RMSNorm needs positive sizes");
  if (hidden % 8 || hidden > 64 * 8 * kNormMaxChunks)
    return set_error(ASPEC_ERR_UNSUPPORTED, "RMSNorm hidden size must be a multiple of 8 up to %d, got %lld",
                     64 * 8 * kNormMaxChunks, (long long)hidden);
  if (!x || !weight || !out || !rstd || (residual && !y_out))
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to RMSNorm forward");
  const void* ptrs[] = {x, residual, weight, y_out, out};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15) return set_error(ASPEC_ERR_INVALID, "RMSNorm needs 16-byte aligned rows");
  NormArgs a = {};
  a.x = static_cast<const uint16_t*>(x);
  a.residual = static_cast<const uint16_t*>(residual);
  a.w = static_cast<const uint16_t*>(weight);
  a.y = static_cast<uint16_t*>(y_out);
  a.out = static_cast<uint16_t*>(out);
  a.rstd = rstd;
  a.rows = rows;
  a.hidden = static_cast<int>(hidden);
  a.eps = eps;
  const dim3 grid(static_cast<uint32_t>((rows + kNormWaves - 1) / kNormWaves));
  hipLaunchKernelGGL(rmsnorm_fwd_kernel, grid, dim3(64 * kNormWaves), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("rmsnorm_fwd_kernel");
}

extern "C" int aspec_rmsnorm_bwd_workspace_bytes(int64_t hidden, size_t* bytes) {
  if (hidden <= 0 || !bytes) return set_error(ASPEC_ERR_INVALID, "workspace size needs a positive hidden size");
  *bytes = static_cast<size_t>(kNormBwdGroups) * static_cast<size_t>(hidden) * sizeof(float);
  return ASPEC_OK;
}

extern "C" int aspec_rmsnorm_bwd(const void* dout, const void* dy_extra, const void* y, const void* weight,
                                 const float* rstd, int64_t rows, int64_t hidden, void* dy,
                                 float* dweight, void* workspace, void* stream) {
  if (rows <= 0 || hidden <= 0) return set_error(ASPEC_ERR_INVALID, "RMSNorm needs positive sizes");
  if (hidden % 8 || hidden > 64 * 8 * kNormMaxChunks)
    return set_error(ASPEC_ERR_UNSUPPORTED, "RMSNorm hidden size must be a multiple of 8 up to %d, got %lld",
                     64 * 8 * kNormMaxChunks, (long long)hidden);
  if (!dout || !y || !weight || !rstd || !dy || !dweight || !workspace)
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to RMSNorm backward");
  const void* ptrs[] = {dout, dy_extra, y, weight, dy, workspace};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15) return set_error(ASPEC_ERR_INVALID, "RMSNorm needs 16-byte aligned rows");
  NormArgs a = {};
  a.dout = static_cast<const uint16_t*>(dout);
  a.dy_extra = static_cast<const uint16_t*>(dy_extra);
  a.y_in = static_cast<const uint16_t*>(y);
  a.w = static_cast<const uint16_t*>(weight);
  a.rstd = const_cast<float*>(rstd);
  a.dy = static_cast<uint16_t*>(dy);
  a.partials = static_cast<float*>(workspace);
  a.dw = dweight;
  a.rows = rows;
  a.hidden = static_cast<int>(hidden);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch ((hidden / 8 + kNormBwdThreads - 1) / kNormBwdThreads) {  // chunks per thread
    case 1: hipLaunchKernelGGL(rmsnorm_bwd_kernel<1>, dim3(kNormBwdGroups), dim3(kNormBwdThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL(rmsnorm_bwd_kernel<2>, dim3(kNormBwdGroups), dim3(kNormBwdThreads), 0, s, a); break;
    case 3: hipLaunchKernelGGL(rmsnorm_bwd_kernel<3>, dim3(kNormBwdGroups), dim3(kNormBwdThreads), 0, s, a); break;
    default: hipLaunchKernelGGL(rmsnorm_bwd_kernel<4>, dim3(kNormBwdGroups), dim3(kNormBwdThreads), 0, s, a); break;
  }
  int rc = check_launch("rmsnorm_bwd_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(column_sum_kernel, dim3(static_cast<uint32_t>((hidden + 63) / 64)), dim3(64 * kColWaves), 0, s,
                     static_cast<const float*>(workspace), kNormBwdGroups, static_cast<int>(hidden),
                     dweight);
  return check_launch("column_sum_kernel");
}

static int swiglu_check(const void* a, const void* b, const void* c, int64_t rows, int64_t ffn) {
  if (rows <= 0 || ffn <= 0) return set_error(ASPEC_ERR_INVALID, "SwiGLU needs positive sizes");
  if (ffn % 8) return set_error(ASPEC_ERR_UNSUPPORTED, "SwiGLU width must be a multiple of 8, got %lld", (long long)ffn);
  if (!a || !b || !c) return set_error(ASPEC_ERR_INVALID, "null pointer passed to SwiGLU");
  const void* ptrs[] = {a, b, c};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15) return set_error(ASPEC_ERR_INVALID, "SwiGLU needs 16-byte aligned rows");
  return ASPEC_OK;
}

extern "C" int aspec_swiglu_fwd(const void* gate_up, int64_t rows, int64_t ffn, void* out, void* stream) {
  int rc = swiglu_check(gate_up, out, out, rows, ffn);
  if (rc) return rc;
  SwiGluArgs a = {};
  a.gu = static_cast<const uint16_t*>(gate_up);
  a.out = static_cast<uint16_t*>(out);
  a.rows = rows;
  a.ffn = ffn;
  const int64_t work = rows * (ffn / 8);
  const dim3 grid(static_cast<uint32_t>(std::min<int64_t>((work + 255) / 256, 256 * 32)));
  hipLaunchKernelGGL(swiglu_fwd_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("swiglu_fwd_kernel");
}

extern "C" int aspec_swiglu_bwd(const void* dout, const void* gate_up, int64_t rows, int64_t ffn,
                                void* dgate_up, void* stream) {
  int rc = swiglu_check(dout, gate_up, dgate_up, rows, ffn);
  if (rc) return rc;
  SwiGluArgs a = {};
  a.gu = static_cast<const uint16_t*>(gate_up);
  a.dout = static_cast<const uint16_t*>(dout);
  a.dgu = static_cast<uint16_t*>(dgate_up);
  a.rows = rows;
  a.ffn = ffn;
  const int64_t work = rows * (ffn / 8);
  const dim3 grid(static_cast<uint32_t>(std::min<int64_t>((work + 255) / 256, 256 * 32)));
  hipLaunchKernelGGL(swiglu_bwd_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("swiglu_bwd_kernel");
}

extern "C" int aspec_adamw_state_bytes(void) { return static_cast<int>(sizeof(AdamState)); }

extern "C" int aspec_adamw_workspace_bytes(size_t* bytes) {
  if (!bytes) return set_error(ASPEC_ERR_INVALID, "null workspace size pointer");
  *bytes = kAdamBlocks * sizeof(float);
  return ASPEC_OK;
}

namespace {

int adamw_launch(void* params, float* master, float* exp_avg, float* exp_avg_sq,
                 const GradTable& table, int64_t n, float lr, float weight_decay, float beta1,
                 float beta2, float eps, float max_grad_norm, void* state, void* workspace,
                 void* stream) {
  if (!params || !master || !exp_avg || !exp_avg_sq || !state || !workspace)
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to AdamW");
  const void* bufs[] = {params, master, exp_avg, exp_avg_sq};
  for (const void* b : bufs)
    if (reinterpret_cast<uintptr_t>(b) & 15)
      return set_error(ASPEC_ERR_INVALID, "AdamW buffers must be 16-byte aligned");
  if (!(beta1 >= 0.f && beta1 < 1.f) || !(beta2 >= 0.f && beta2 < 1.f) || !(eps >= 0.f))
    return set_error(ASPEC_ERR_INVALID, "AdamW betas must lie in [0, 1) and eps must be non-negative");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* partials = static_cast<float*>(workspace);
  AdamState* st = static_cast<AdamState*>(state);
  hipLaunchKernelGGL(grad_sumsq_kernel, dim3(kAdamBlocks), dim3(256), 0, s, table, n, partials);
  int rc = check_launch("grad_sumsq_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(adam_finalize_kernel, dim3(1), dim3(64), 0, s, static_cast<const float*>(partials),
                     kAdamBlocks, max_grad_norm, beta1, beta2, table.nseg, table.active, st);
  if ((rc = check_launch("adam_finalize_kernel"))) return rc;
  AdamArgs a = {};
  a.param = static_cast<uint16_t*>(params);
  a.master = master;
  a.m = exp_avg;
  a.v = exp_avg_sq;
  a.grad = table;
  a.n = n;
  a.lr = lr;
  a.wd = weight_decay;
  a.b1 = beta1;
  a.b2 = beta2;
  a.eps = eps;
  a.st = st;
  const dim3 grid(static_cast<uint32_t>(std::min<int64_t>((n / 8 + 255) / 256 + 1, 256 * 16)));
  hipLaunchKernelGGL(adam_update_kernel, grid, dim3(256), 0, s, a);
  return check_launch("adam_update_kernel");
}

}  // namespace

extern "C" int aspec_adamw_step(void* params, float* master, float* exp_avg, float* exp_avg_sq,
                                const void* grads, int64_t n, float lr, float weight_decay,
                                float beta1, float beta2, float eps, float max_grad_norm,
                                void* state, void* workspace, void* stream) {
  if (n <= 0) return set_error(ASPEC_ERR_INVALID, "AdamW needs a positive parameter count");
  if (!grads) return set_error(ASPEC_ERR_INVALID, "null pointer passed to AdamW");
  if (reinterpret_cast<uintptr_t>(grads) & 15)
    return set_error(ASPEC_ERR_INVALID, "AdamW buffers must be 16-byte aligned");
  GradTable t = {};
  t.nseg = 1;
  t.active = 1;
  t.end[0] = n;
  t.ptr[0] = static_cast<const uint16_t*>(grads);
  return adamw_launch(params, master, exp_avg, exp_avg_sq, t, n, lr, weight_decay, beta1, beta2,
                      eps, max_grad_norm, state, workspace, stream);
}

extern "C" int aspec_adamw_step_segments(void* params, float* master, float* exp_avg,
                                         float* exp_avg_sq, const void* const* seg_grads,
                                         const int64_t* seg_numel, int nseg, float lr,
                                         float weight_decay, float beta1, float beta2, float eps,
                                         float max_grad_norm, void* state, void* workspace,
                                         void* stream) {
  if (!seg_grads || !seg_numel) return set_error(ASPEC_ERR_INVALID, "null segment table passed to AdamW");
  if (nseg <= 0 || nseg > kMaxGradSegments)
    return set_error(ASPEC_ERR_UNSUPPORTED, "AdamW segment count must lie in [1, %d], got %d",
                     kMaxGradSegments, nseg);
  GradTable t = {};
  t.nseg = nseg;
  int64_t n = 0;
  for (int i = 0; i < nseg; ++i) {
    if (seg_numel[i] <= 0)
      return set_error(ASPEC_ERR_INVALID, "AdamW segment %d has no elements", i);
    if (i + 1 < nseg && (seg_numel[i] & 7))
      return set_error(ASPEC_ERR_INVALID,
                       "AdamW segment %d holds %lld elements: every segment but the last must hold "
                       "a multiple of 8", i, static_cast<long long>(seg_numel[i]));
    if (reinterpret_cast<uintptr_t>(seg_grads[i]) & 15)
      return set_error(ASPEC_ERR_INVALID, "AdamW segment %d gradient must be 16-byte aligned", i);
    n += seg_numel[i];
    t.end[i] = n;
    t.ptr[i] = static_cast<const uint16_t*>(seg_grads[i]);
    if (seg_grads[i]) t.active |= 1ull << i;
  }
  return adamw_launch(params, master, exp_avg, exp_avg_sq, t, n, lr, weight_decay, beta1, beta2,
                      eps, max_grad_norm, state, workspace, stream);
}
