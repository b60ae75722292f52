// DSpark Q/K preparation: per-head RMSNorm, the context/draft key join and indexed RoPE, forward
// and backward (aspec/models/ops/dspark_qk_norm_rope.py:134-419; eager definition
// aspec/models/draft/dflash.py:280-327). HBM-bound elementwise work over head rows of 128 dims.
//
// Forward, per head row x (one token, one head): rstd = 1/sqrt(mean(x^2) + eps), a = x*rstd*w,
// out = a*cos[pos] + rotate_half(a)*sin[pos]; all in fp32, rounded once to bf16 or fp16. Query rows take
// the query weight; context and draft key rows take the key weight and land in one joined key
// tensor [B, Lc + Ld, Hkv, D] (context first).
// Backward, with g = dL/dout: da = g*cos + rotate_half^T(g*sin), dw += da*n (n = x*rstd),
// dn = da*w, dx = rstd*(dn - n*mean(dn*n)). dw is fp32, reduced per workgroup and then over
// workgroups in a fixed order (deterministic).
//
// Lane layout: 16 lanes per head row; lane j holds dims 4j..4j+3 and 64+4j..64+4j+3, so
// rotate_half pairs stay inside one lane. A 256-thread workgroup covers 16 head rows.
#include <mutex>

#include "common.h"

namespace aspec {
namespace {

constexpr int kQkDim = 128;
constexpr int kRowsPerGroup = 16;            // head rows per 256-thread workgroup
constexpr int kBwdMaxGroups = 2048;          // backward grid cap (fixed: deterministic dw)

struct QkArgs {
  const uint16_t* query;  // [B*Ld, Hq, D]
  const uint16_t* ctx;    // [B*Lc, Hkv, D]
  const uint16_t* draft;  // [B*Ld, Hkv, D]
  const uint16_t* wq;
  const uint16_t* wk;
  const uint16_t* cos;    // [rope_rows, rope_stride]
  const uint16_t* sin;
  int64_t rope_rows, rope_stride;
  const int64_t* pos_q;    // [B*Ld]
  const int64_t* pos_ctx;  // [B*Lc]
  const int64_t* pos_draft;
  int64_t batch, lc, ld, hq, hkv;
  float eps;
  uint16_t* q_out;  // [B*Ld, Hq, D] (forward) / dquery (backward)
  uint16_t* k_out;  // [B*(Lc+Ld), Hkv, D] (forward)
  uint16_t* dctx;   // backward
  uint16_t* ddraft;
  const uint16_t* gq;  // backward: dL/dq_out, dL/dk_out
  const uint16_t* gk;
  float* rstd_q;  // [B*Ld, Hq]
  float* rstd_k;  // [B*(Lc+Ld), Hkv]
  float* partials;  // backward: [2][groups][D]
  float* dwq;
  float* dwk;
  int32_t* flags;  // bit 0: a position outside the cos/sin table
  int64_t rows_q, rows_c, rows_d;  // head rows per segment
};

// Where head row r lives: segment (0 query, 1 context key, 2 draft key), its source / output
// element offsets, rstd index, position pointer.
struct HeadRow {
  int seg;
  int64_t src, out, rstd, token;
};

__device__ __forceinline__ HeadRow locate(const QkArgs& a, int64_t r) {
  HeadRow h;
  if (r < a.rows_q) {
    h.seg = 0;
    h.token = r / a.hq;
    h.src = r * kQkDim;
    h.out = h.src;
    h.rstd = r;
    return h;
  }
  r -= a.rows_q;
  const bool is_ctx = r < a.rows_c;
  if (!is_ctx) r -= a.rows_c;
  const int64_t seg_len = is_ctx ? a.lc : a.ld;
  const int64_t token = r / a.hkv;
  const int64_t head = r - token * a.hkv;
  const int64_t b = token / seg_len;
  const int64_t t = token - b * seg_len;
  const int64_t out_row = b * (a.lc + a.ld) + (is_ctx ? 0 : a.lc) + t;
  h.seg = is_ctx ? 1 : 2;
  h.token = token;
  h.src = r * kQkDim;
  h.out = (out_row * a.hkv + head) * kQkDim;
  h.rstd = out_row * a.hkv + head;
  return h;
}

// Activations, weights and cos/sin are bf16 or fp16 (F16); arithmetic is fp32 and each output is
// rounded once, to nearest even.
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <bool F16>
__device__ __forceinline__ void load4(const uint16_t* p, float (&v)[4]) {
  const u32x2 w = *reinterpret_cast<const u32x2*>(p);
  if constexpr (F16) {
    v[0] = f16_to_f32(w.x & 0xffffu);
    v[1] = f16_to_f32(w.x >> 16);
    v[2] = f16_to_f32(w.y & 0xffffu);
    v[3] = f16_to_f32(w.y >> 16);
  } else {
    v[0] = __uint_as_float(w.x << 16);
    v[1] = __uint_as_float(w.x & 0xffff0000u);
    v[2] = __uint_as_float(w.y << 16);
    v[3] = __uint_as_float(w.y & 0xffff0000u);
  }
}

template <bool F16>
__device__ __forceinline__ void store4(uint16_t* p, const float (&v)[4]) {
  u32x2 w;
  if constexpr (F16) {
    w.x = f32_to_f16_bits(v[0]) | (f32_to_f16_bits(v[1]) << 16);
    w.y = f32_to_f16_bits(v[2]) | (f32_to_f16_bits(v[3]) << 16);
  } else {
    w.x = pack_bf16x2(v[0], v[1]);
    w.y = pack_bf16x2(v[2], v[3]);
  }
  *reinterpret_cast<u32x2*>(p) = w;
}

// Sum over the 16 lanes of one head row.
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// cos / sin of this lane's dims at `pos` (clamped into the table; `bad` when it was outside).
template <bool F16>
__device__ __forceinline__ void rope_rows(const QkArgs& a, int64_t pos, int j, float (&cl)[4],
                                          float (&ch)[4], float (&sl)[4], float (&sh)[4],
                                          bool& bad) {
  bad = pos < 0 || pos >= a.rope_rows;
  const int64_t p = bad ? 0 : pos;
  const uint16_t* c = a.cos + p * a.rope_stride;
  const uint16_t* s = a.sin + p * a.rope_stride;
  load4<F16>(c + 4 * j, cl);
  load4<F16>(c + 64 + 4 * j, ch);
  load4<F16>(s + 4 * j, sl);
  load4<F16>(s + 64 + 4 * j, sh);
}

template <bool F16>
__global__ void __launch_bounds__(256) qk_norm_rope_fwd_kernel(QkArgs a) {
  const int j = threadIdx.x & 15;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowsPerGroup + (threadIdx.x >> 4);
  if (r >= a.rows_q + a.rows_c + a.rows_d) return;  // whole 16-lane groups exit together
  const HeadRow h = locate(a, r);
  const uint16_t* src = (h.seg == 0 ? a.query : h.seg == 1 ? a.ctx : a.draft) + h.src;
  const int64_t* pos = h.seg == 0 ? a.pos_q : h.seg == 1 ? a.pos_ctx : a.pos_draft;
  const uint16_t* w = h.seg == 0 ? a.wq : a.wk;
  float xl[4], xh[4], wl[4], wh[4];
  load4<F16>(src + 4 * j, xl);
  load4<F16>(src + 64 + 4 * j, xh);
  load4<F16>(w + 4 * j, wl);
  load4<F16>(w + 64 + 4 * j, wh);
  float cl[4], ch[4], sl[4], sh[4];
  bool bad;
  rope_rows<F16>(a, pos[h.token], j, cl, ch, sl, sh, bad);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += xl[i] * xl[i] + xh[i] * xh[i];
  const float rstd = rsqrtf(row_sum(ss) * (1.f / kQkDim) + a.eps);
  float ol[4], oh[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float al = xl[i] * rstd * wl[i];
    const float ah = xh[i] * rstd * wh[i];
    ol[i] = bad ? NAN : al * cl[i] - ah * sl[i];
    oh[i] = bad ? NAN : ah * ch[i] + al * sh[i];
  }
  uint16_t* dst = (h.seg == 0 ? a.q_out : a.k_out) + h.out;
  store4<F16>(dst + 4 * j, ol);
  store4<F16>(dst + 64 + 4 * j, oh);
  if (j == 0) {
    (h.seg == 0 ? a.rstd_q : a.rstd_k)[h.rstd] = rstd;
    if (bad) atomicOr(a.flags, 1);
  }
}

// Grid-strided over 16-row groups; per-lane dw accumulators for both weights, reduced over the
// workgroup into partials[seg][blockIdx][D].
template <bool F16>
__global__ void __launch_bounds__(256) qk_norm_rope_bwd_kernel(QkArgs a) {
  __shared__ float red[2][kRowsPerGroup][kQkDim];
  const int j = threadIdx.x & 15;
  const int grp = threadIdx.x >> 4;
  const int64_t total = a.rows_q + a.rows_c + a.rows_d;
  float dq_l[4] = {}, dq_h[4] = {}, dk_l[4] = {}, dk_h[4] = {};
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kRowsPerGroup + grp; r < total;
       r += static_cast<int64_t>(gridDim.x) * kRowsPerGroup) {
    const HeadRow h = locate(a, r);
    const uint16_t* src = (h.seg == 0 ? a.query : h.seg == 1 ? a.ctx : a.draft) + h.src;
    const uint16_t* g = (h.seg == 0 ? a.gq : a.gk) + h.out;
    const int64_t* pos = h.seg == 0 ? a.pos_q : h.seg == 1 ? a.pos_ctx : a.pos_draft;
    const uint16_t* w = h.seg == 0 ? a.wq : a.wk;
    float xl[4], xh[4], gl[4], gh[4], wl[4], wh[4];
    load4<F16>(src + 4 * j, xl);
    load4<F16>(src + 64 + 4 * j, xh);
    load4<F16>(g + 4 * j, gl);
    load4<F16>(g + 64 + 4 * j, gh);
    load4<F16>(w + 4 * j, wl);
    load4<F16>(w + 64 + 4 * j, wh);
    float cl[4], ch[4], sl[4], sh[4];
    bool bad;
    rope_rows<F16>(a, pos[h.token], j, cl, ch, sl, sh, bad);
    const float rstd = (h.seg == 0 ? a.rstd_q : a.rstd_k)[h.rstd];
    float nl[4], nh[4], dnl[4], dnh[4];
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      nl[i] = xl[i] * rstd;
      nh[i] = xh[i] * rstd;
      // transpose of out = a*cos + rotate_half(a)*sin
      const float dal = bad ? NAN : gl[i] * cl[i] + gh[i] * sh[i];
      const float dah = bad ? NAN : gh[i] * ch[i] - gl[i] * sl[i];
      if (h.seg == 0) {
        dq_l[i] += dal * nl[i];
        dq_h[i] += dah * nh[i];
      } else {
        dk_l[i] += dal * nl[i];
        dk_h[i] += dah * nh[i];
      }
      dnl[i] = dal * wl[i];
      dnh[i] = dah * wh[i];
      dot += dnl[i] * nl[i] + dnh[i] * nh[i];
    }
    const float mean = row_sum(dot) * (1.f / kQkDim);
    float ol[4], oh[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ol[i] = rstd * (dnl[i] - nl[i] * mean);
      oh[i] = rstd * (dnh[i] - nh[i] * mean);
    }
    uint16_t* dst = (h.seg == 0 ? a.q_out : h.seg == 1 ? a.dctx : a.ddraft) + h.src;
    store4<F16>(dst + 4 * j, ol);
    store4<F16>(dst + 64 + 4 * j, oh);
    if (j == 0 && bad) atomicOr(a.flags, 1);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    red[0][grp][4 * j + i] = dq_l[i];
    red[0][grp][64 + 4 * j + i] = dq_h[i];
    red[1][grp][4 * j + i] = dk_l[i];
    red[1][grp][64 + 4 * j + i] = dk_h[i];
  }
  __syncthreads();
  const int seg = threadIdx.x >> 7;  // 256 threads: (weight, dim)
  const int d = threadIdx.x & 127;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kRowsPerGroup; ++k) s += red[seg][k][d];
  a.partials[(static_cast<int64_t>(seg) * gridDim.x + blockIdx.x) * kQkDim + d] = s;
}

// dw[seg][d] = sum over workgroups of partials[seg][b][d]: one workgroup per (seg, d), each
// thread summing a strided slice, then a fixed-order tree over the threads (deterministic).
__global__ void __launch_bounds__(256) qk_norm_rope_dw_kernel(QkArgs a, int groups) {
  __shared__ float part[256];
  const int seg = blockIdx.x / kQkDim;
  const int d = blockIdx.x % kQkDim;
  const float* p = a.partials + static_cast<int64_t>(seg) * groups * kQkDim + d;
  float s = 0.f;
  for (int b = threadIdx.x; b < groups; b += 256) s += p[static_cast<int64_t>(b) * kQkDim];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int width = 128; width > 0; width >>= 1) {
    if (threadIdx.x < width) part[threadIdx.x] += part[threadIdx.x + width];
    __syncthreads();
  }
  if (threadIdx.x == 0) (seg == 0 ? a.dwq : a.dwk)[d] = part[0];
}

int check_dtype(int32_t dtype) {
  if (dtype != ASPEC_MASK_BF16 && dtype != ASPEC_MASK_F16)
    return set_error(ASPEC_ERR_UNSUPPORTED, "DSpark Q/K norm+RoPE serves bf16 and fp16 (dtype %d)", dtype);
  return ASPEC_OK;
}

int check_sizes(const QkArgs& a, int64_t head_dim) {
  if (head_dim != kQkDim)
    return set_error(ASPEC_ERR_UNSUPPORTED, "DSpark Q/K norm+RoPE supports head_dim 128 only, got %lld",
                     (long long)head_dim);
  if (a.batch <= 0 || a.lc < 0 || a.ld <= 0 || a.hq <= 0 || a.hkv <= 0)
    return set_error(ASPEC_ERR_INVALID, "DSpark Q/K norm+RoPE needs positive batch, draft length and heads");
  if (a.rope_rows <= 0 || a.rope_stride < kQkDim)
    return set_error(ASPEC_ERR_INVALID, "cos/sin tables need at least one row of head_dim values");
  const void* ptrs[] = {a.query, a.draft, a.wq, a.wk, a.cos, a.sin};
  for (const void* p : ptrs)
    if (!p) return set_error(ASPEC_ERR_INVALID, "null pointer passed to DSpark Q/K norm+RoPE");
  if (a.lc > 0 && !a.ctx) return set_error(ASPEC_ERR_INVALID, "null context key with a nonempty context");
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.query) | reinterpret_cast<uintptr_t>(a.draft) |
                          reinterpret_cast<uintptr_t>(a.ctx) | reinterpret_cast<uintptr_t>(a.wq) |
                          reinterpret_cast<uintptr_t>(a.wk) | reinterpret_cast<uintptr_t>(a.cos) |
                          reinterpret_cast<uintptr_t>(a.sin);
  if ((align & 7) || (a.rope_stride & 3))
    return set_error(ASPEC_ERR_INVALID, "DSpark Q/K norm+RoPE needs 8-byte aligned rows");
  return ASPEC_OK;
}

QkArgs make_args(const void* query, const void* context_key, const void* draft_key,
                 const void* q_weight, const void* k_weight, const void* cos, const void* sin,
                 int64_t rope_rows, int64_t rope_stride, const int64_t* pos_q,
                 const int64_t* pos_ctx, const int64_t* pos_draft, int64_t batch,
                 int64_t context_len, int64_t draft_len, int64_t q_heads, int64_t kv_heads,
                 float eps) {
  QkArgs a = {};
  a.query = static_cast<const uint16_t*>(query);
  a.ctx = static_cast<const uint16_t*>(context_key);
  a.draft = static_cast<const uint16_t*>(draft_key);
  a.wq = static_cast<const uint16_t*>(q_weight);
  a.wk = static_cast<const uint16_t*>(k_weight);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.rope_rows = rope_rows;
  a.rope_stride = rope_stride;
  a.pos_q = pos_q;
  a.pos_ctx = pos_ctx;
  a.pos_draft = pos_draft;
  a.batch = batch;
  a.lc = context_len;
  a.ld = draft_len;
  a.hq = q_heads;
  a.hkv = kv_heads;
  a.eps = eps;
  a.rows_q = batch * draft_len * q_heads;
  a.rows_c = batch * context_len * kv_heads;
  a.rows_d = batch * draft_len * kv_heads;
  return a;
}

int bwd_groups(const QkArgs& a) {
  const int64_t groups = (a.rows_q + a.rows_c + a.rows_d + kRowsPerGroup - 1) / kRowsPerGroup;
  return static_cast<int>(groups < kBwdMaxGroups ? groups : kBwdMaxGroups);
}

}  // namespace

// Scratch of aspec_qk_norm_rope_bwd_noalloc: the per-workgroup weight-gradient partials of one
// call, [2][groups][128] fp32 with groups <= kBwdMaxGroups, so 2 MiB covers every size. Each GPU
// the library runs on holds its own copy until the process ends. Every slot a call reads is
// written earlier in the same call, so nothing needs clearing between calls; calls that overlap
// on one GPU share the array and race.
static __device__ __align__(256) float scratch[2 * kBwdMaxGroups * kQkDim];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of `scratch` on the current device, looked up once per device (no
// allocation: the array is part of the loaded code object).
int scratch_on_current_device(float** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess)
    return set_error(ASPEC_ERR_RUNTIME, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxScratchDevices)
    return set_error(ASPEC_ERR_UNSUPPORTED, "device %d beyond the %d scratch slots", device,
                     kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return set_error(ASPEC_ERR_RUNTIME, "hipGetSymbolAddress(scratch) failed on device %d: %s",
                       device, hipGetErrorString(err));
    g_scratch_ptr[device] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[device];
  return ASPEC_OK;
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_qk_norm_rope_fwd(const void* query, const void* context_key,
                                      const void* draft_key, const void* q_weight,
                                      const void* k_weight, const void* cos, const void* sin,
                                      int64_t rope_rows, int64_t rope_stride,
                                      const int64_t* query_positions,
                                      const int64_t* context_positions,
                                      const int64_t* draft_positions, int64_t batch,
                                      int64_t context_len, int64_t draft_len, int64_t q_heads,
                                      int64_t kv_heads, int64_t head_dim, float eps, int32_t dtype,
                                      void* q_out, void* k_out, float* rstd_q, float* rstd_k,
                                      int32_t* status_flags, void* stream) {
  if (int rc0 = check_dtype(dtype)) return rc0;
  QkArgs a = make_args(query, context_key, draft_key, q_weight, k_weight, cos, sin, rope_rows,
                       rope_stride, query_positions, context_positions, draft_positions, batch,
                       context_len, draft_len, q_heads, kv_heads, eps);
  int rc = check_sizes(a, head_dim);
  if (rc) return rc;
  if (!q_out || !k_out || !rstd_q || !rstd_k || !status_flags || !query_positions ||
      !draft_positions || (context_len > 0 && !context_positions))
    return set_error(ASPEC_ERR_INVALID, "null output, rstd, position or status pointer");
  if (((reinterpret_cast<uintptr_t>(q_out) | reinterpret_cast<uintptr_t>(k_out)) & 7))
    return set_error(ASPEC_ERR_INVALID, "DSpark Q/K norm+RoPE needs 8-byte aligned rows");
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_out = static_cast<uint16_t*>(k_out);
  a.rstd_q = rstd_q;
  a.rstd_k = rstd_k;
  a.flags = status_flags;
  const int64_t groups = (a.rows_q + a.rows_c + a.rows_d + kRowsPerGroup - 1) / kRowsPerGroup;
  if (dtype == ASPEC_MASK_F16)
    hipLaunchKernelGGL(qk_norm_rope_fwd_kernel<true>, dim3(static_cast<uint32_t>(groups)), dim3(256),
                       0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(qk_norm_rope_fwd_kernel<false>, dim3(static_cast<uint32_t>(groups)), dim3(256),
                       0, static_cast<hipStream_t>(stream), a);
  return check_launch("qk_norm_rope_fwd_kernel");
}

extern "C" int aspec_qk_norm_rope_bwd_workspace_bytes(int64_t batch, int64_t context_len,
                                                      int64_t draft_len, int64_t q_heads,
                                                      int64_t kv_heads, size_t* bytes) {
  if (batch <= 0 || context_len < 0 || draft_len <= 0 || q_heads <= 0 || kv_heads <= 0 || !bytes)
    return set_error(ASPEC_ERR_INVALID, "workspace size needs positive sizes");
  QkArgs a = {};
  a.rows_q = batch * draft_len * q_heads;
  a.rows_c = batch * context_len * kv_heads;
  a.rows_d = batch * draft_len * kv_heads;
  *bytes = static_cast<size_t>(2) * bwd_groups(a) * kQkDim * sizeof(float);
  return ASPEC_OK;
}

extern "C" int aspec_qk_norm_rope_bwd(
    const void* grad_q, const void* grad_k, const void* query, const void* context_key,
    const void* draft_key, const float* rstd_q, const float* rstd_k, const void* q_weight,
    const void* k_weight, const void* cos, const void* sin, int64_t rope_rows,
    int64_t rope_stride, const int64_t* query_positions, const int64_t* context_positions,
    const int64_t* draft_positions, int64_t batch, int64_t context_len, int64_t draft_len,
    int64_t q_heads, int64_t kv_heads, int64_t head_dim, float eps, int32_t dtype, void* d_query,
    void* d_context_key, void* d_draft_key, float* dw_q, float* dw_k, void* workspace,
    int32_t* status_flags, void* stream) {
  if (int rc0 = check_dtype(dtype)) return rc0;
  QkArgs a = make_args(query, context_key, draft_key, q_weight, k_weight, cos, sin, rope_rows,
                       rope_stride, query_positions, context_positions, draft_positions, batch,
                       context_len, draft_len, q_heads, kv_heads, eps);
  int rc = check_sizes(a, head_dim);
  if (rc) return rc;
  if (!grad_q || !grad_k || !rstd_q || !rstd_k || !d_query || !d_draft_key || !dw_q || !dw_k ||
      !workspace || !status_flags || !query_positions || !draft_positions ||
      (context_len > 0 && (!context_positions || !d_context_key)))
    return set_error(ASPEC_ERR_INVALID, "null gradient, rstd, position, workspace or status pointer");
  if (((reinterpret_cast<uintptr_t>(grad_q) | reinterpret_cast<uintptr_t>(grad_k) |
        reinterpret_cast<uintptr_t>(d_query) | reinterpret_cast<uintptr_t>(d_context_key) |
        reinterpret_cast<uintptr_t>(d_draft_key)) & 7))
    return set_error(ASPEC_ERR_INVALID, "DSpark Q/K norm+RoPE needs 8-byte aligned rows");
  a.gq = static_cast<const uint16_t*>(grad_q);
  a.gk = static_cast<const uint16_t*>(grad_k);
  a.rstd_q = const_cast<float*>(rstd_q);
  a.rstd_k = const_cast<float*>(rstd_k);
  a.q_out = static_cast<uint16_t*>(d_query);
  a.dctx = static_cast<uint16_t*>(d_context_key);
  a.ddraft = static_cast<uint16_t*>(d_draft_key);
  a.dwq = dw_q;
  a.dwk = dw_k;
  a.partials = static_cast<float*>(workspace);
  a.flags = status_flags;
  const int groups = bwd_groups(a);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASPEC_MASK_F16)
    hipLaunchKernelGGL(qk_norm_rope_bwd_kernel<true>, dim3(static_cast<uint32_t>(groups)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(qk_norm_rope_bwd_kernel<false>, dim3(static_cast<uint32_t>(groups)), dim3(256), 0, s, a);
  if ((rc = check_launch("qk_norm_rope_bwd_kernel"))) return rc;
  hipLaunchKernelGGL(qk_norm_rope_dw_kernel, dim3(2 * kQkDim), dim3(256), 0, s, a, groups);
  return check_launch("qk_norm_rope_dw_kernel");
}

extern "C" int aspec_qk_norm_rope_bwd_noalloc(
    const void* grad_q, const void* grad_k, const void* query, const void* context_key,
    const void* draft_key, const float* rstd_q, const float* rstd_k, const void* q_weight,
    const void* k_weight, const void* cos, const void* sin, int64_t rope_rows,
    int64_t rope_stride, const int64_t* query_positions, const int64_t* context_positions,
    const int64_t* draft_positions, int64_t batch, int64_t context_len, int64_t draft_len,
    int64_t q_heads, int64_t kv_heads, int64_t head_dim, float eps, int32_t dtype, void* d_query,
    void* d_context_key, void* d_draft_key, float* dw_q, float* dw_k, int32_t* status_flags,
    void* stream) {
  size_t need = 0;
  int rc = aspec_qk_norm_rope_bwd_workspace_bytes(batch, context_len, draft_len, q_heads, kv_heads,
                                                  &need);
  if (rc) return rc;
  if (need > sizeof(scratch))
    return set_error(ASPEC_ERR_UNSUPPORTED,
                     "Q/K norm+RoPE backward needs %zu bytes of scratch; the static scratch holds %zu",
                     need, sizeof(scratch));
  float* ptr = nullptr;
  if ((rc = scratch_on_current_device(&ptr))) return rc;
  return aspec_qk_norm_rope_bwd(grad_q, grad_k, query, context_key, draft_key, rstd_q, rstd_k,
                                q_weight, k_weight, cos, sin, rope_rows, rope_stride,
                                query_positions, context_positions, draft_positions, batch,
                                context_len, draft_len, q_heads, kv_heads, head_dim, eps, dtype,
                                d_query, d_context_key, d_draft_key, dw_q, dw_k, ptr, status_flags,
                                stream);
}
