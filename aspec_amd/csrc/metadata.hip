// THD integer metadata on the GPU: the eight mask tensors, per-row interval endpoints, tile classes
// and the ordered / transposed tile lists. All integer work, HBM- and latency-bound.
#include "common.h"
#include "plan.h"

namespace aspec {
namespace {

constexpr int64_t kInt64Max = 0x7fffffffffffffffLL;

__device__ __forceinline__ int64_t sortable_doc(int64_t d) { return d >= 0 ? d : kInt64Max; }

// torch.searchsorted(right=False): first index i with a[i] >= v.
__device__ __forceinline__ int64_t lower_bound(const int64_t* a, int64_t n, int64_t v) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (a[mid] < v) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Same over the "sortable" document ids (negative padding ids mapped past every document),
// direct_cp.py:817-825. upper=true gives searchsorted(right=True).
__device__ __forceinline__ int64_t doc_bound(const int64_t* docs, int64_t n, int64_t v, bool upper) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    int64_t x = sortable_doc(docs[mid]);
    bool go_right = upper ? (x <= v) : (x < v);
    if (go_right) lo = mid + 1; else hi = mid;
  }
  return lo;
}

struct RowArgs {
  const int64_t* anchors;
  const uint8_t* keep;
  const int64_t* anchor_docs;
  const int64_t* ctx_pos;
  const int64_t* ctx_docs;
  int64_t num_blocks, block, T, seq_len, ctx_window, q_window;
  int causal;
  int32_t* qaux;
  int32_t* kaux;
  int32_t* ends;
  int32_t* flags;
};

// One thread per query row q (which also owns draft key T+q, the same block and offset at CP=1),
// followed by one thread per context key; blockIdx.y is the batch row b. Inputs are [batch][...]
// contiguous; outputs are the rows of all batch rows back to back: query_aux [4][B*Nq], key_aux
// [4][B*K], endpoints [5][B*Nq] in the flattened key space (row b's keys are b*K .. b*K + K - 1;
// dropped rows stay all zero), so one attention launch covers every batch row.
__global__ void row_metadata_kernel(RowArgs a) {
  const int64_t nq = a.num_blocks * a.block;
  const int64_t K = a.T + nq;
  const int64_t b = blockIdx.y;
  const int64_t nb = gridDim.y;
  a.anchors += b * a.num_blocks;
  a.keep += b * a.num_blocks;
  a.anchor_docs += b * a.num_blocks;
  a.ctx_pos += b * a.T;
  a.ctx_docs += b * a.T;
  const int64_t qrow0 = b * nq;   // this batch row's first flattened query row
  const int64_t key0 = b * K;     // and first flattened key
  const int64_t NQ = nb * nq;     // flattened field strides
  const int64_t NK = nb * K;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid < nq) {
    const int64_t q = tid;
    const int64_t r = q / a.block;
    const int64_t o = q - r * a.block;
    const int64_t anchor = a.anchors[r];
    const int64_t doc = a.anchor_docs[r];
    const bool block_keep = a.keep[r] != 0;
    // _token_keep (direct_cp.py:370-379) and _query_metadata (thd_attention.py:25-39).
    const bool token_keep = block_keep && (a.seq_len <= 0 || anchor + o < a.seq_len);
    const bool query_keep = token_keep && doc >= 0;
    if (a.qaux) {
      a.qaux[0 * NQ + qrow0 + q] = static_cast<int32_t>(anchor);
      a.qaux[1 * NQ + qrow0 + q] = query_keep ? 1 : 0;
      a.qaux[2 * NQ + qrow0 + q] = static_cast<int32_t>(r);
      a.qaux[3 * NQ + qrow0 + q] = static_cast<int32_t>(doc);
    }
    if (a.kaux) {  // _key_metadata draft half (thd_attention.py:42-56)
      const int64_t kq = key0 + a.T + q;
      a.kaux[0 * NK + kq] = static_cast<int32_t>(doc);
      a.kaux[1 * NK + kq] = static_cast<int32_t>(-o - 1);
      a.kaux[2 * NK + kq] = static_cast<int32_t>(r);
      a.kaux[3 * NK + kq] = query_keep ? 1 : 0;
    }
    if (a.ends) {  // _build_cudnn_thd_mask (direct_cp.py:790-878)
      int64_t cb = 0, ce = 0, db = 0, de = 0;
      if (query_keep) {
        int64_t lower = 0;
        if (a.ctx_window > 0) lower = max(lower, anchor - a.ctx_window);
        if (a.q_window > 0) lower = max(lower, anchor + o - a.q_window + 1);
        cb = lower_bound(a.ctx_pos, a.T, lower);
        ce = lower_bound(a.ctx_pos, a.T, anchor);
        const int64_t sd = sortable_doc(doc);
        cb = max(cb, doc_bound(a.ctx_docs, a.T, sd, false));
        ce = min(ce, doc_bound(a.ctx_docs, a.T, sd, true));
        cb = min(cb, ce);
        const int64_t base = a.T + r * a.block;
        int64_t valid = a.block;
        if (a.seq_len > 0) valid = min(max(a.seq_len - anchor, (int64_t)0), a.block);
        db = base;
        de = base + valid;
        if (a.causal) de = min(de, base + o + 1);
        if (a.q_window > 0) {
          db = base + max(o - a.q_window + 1, (int64_t)0);
          de = min(de, base + min(o + a.q_window, a.block));
        }
        db = min(db, de);
        cb += key0;
        ce += key0;
        db += key0;
        de += key0;
      }
      a.ends[0 * NQ + qrow0 + q] = 0;
      a.ends[1 * NQ + qrow0 + q] = static_cast<int32_t>(cb);
      a.ends[2 * NQ + qrow0 + q] = static_cast<int32_t>(ce);
      a.ends[3 * NQ + qrow0 + q] = static_cast<int32_t>(db);
      a.ends[4 * NQ + qrow0 + q] = static_cast<int32_t>(de);
    }
  } else if (tid < nq + a.T) {
    const int64_t t = tid - nq;
    const int64_t doc = a.ctx_docs[t];
    if (a.kaux) {  // _key_metadata context half
      a.kaux[0 * NK + key0 + t] = static_cast<int32_t>(doc);
      a.kaux[1 * NK + key0 + t] = static_cast<int32_t>(a.ctx_pos[t]);
      a.kaux[2 * NK + key0 + t] = -1;
      a.kaux[3 * NK + key0 + t] = doc >= 0 ? 1 : 0;
    }
    if (a.flags && t > 0) {
      int bad = 0;
      if (a.ctx_pos[t] < a.ctx_pos[t - 1]) bad |= 1;
      if (sortable_doc(doc) < sortable_doc(a.ctx_docs[t - 1])) bad |= 2;
      if (bad) atomicOr(a.flags, bad);
    }
  }
}

// One context-parallel rank's partial (direct_cp.py:750-878 with cp_size > 1): every query row of
// the collective block order against this rank's keys, its context shard (ascending positions)
// followed by the draft keys of its own blocks. Query block rc is block query_blocks[rc]; its draft
// keys are those of local slot j when local_blocks[j] is that block (local_blocks ascending), and
// otherwise absent: both draft endpoints are the key length K_local, as the reference writes them.
struct ShardArgs {
  const int64_t* anchors;      // [batch][num_blocks], original block order
  const uint8_t* keep;
  const int64_t* anchor_docs;
  const int64_t* ctx_pos;      // [batch][T] this rank's context positions
  const int64_t* ctx_docs;
  const int64_t* query_blocks;  // [nqb] collective order
  const int64_t* local_blocks;  // [nlb] ascending
  int64_t num_blocks, nqb, nlb, block, T, seq_len, ctx_window, q_window;
  int causal;
  int32_t* ends;  // [5][batch * nqb * block]
  int32_t* flags;
};

__global__ void shard_endpoints_kernel(ShardArgs a) {
  const int64_t nq = a.nqb * a.block;
  const int64_t K = a.T + a.nlb * a.block;
  const int64_t b = blockIdx.y;
  const int64_t NQ = static_cast<int64_t>(gridDim.y) * nq;
  a.anchors += b * a.num_blocks;
  a.keep += b * a.num_blocks;
  a.anchor_docs += b * a.num_blocks;
  a.ctx_pos += b * a.T;
  a.ctx_docs += b * a.T;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid < nq) {
    const int64_t q = tid;
    const int64_t rc = q / a.block;
    const int64_t o = q - rc * a.block;
    const int64_t r = a.query_blocks[rc];
    if (r < 0 || r >= a.num_blocks) {
      atomicOr(a.flags, 4);
      for (int e = 0; e < 5; ++e) a.ends[e * NQ + b * nq + q] = 0;
      return;
    }
    const int64_t anchor = a.anchors[r];
    const int64_t doc = a.anchor_docs[r];
    const bool token_keep = a.keep[r] != 0 && (a.seq_len <= 0 || anchor + o < a.seq_len);
    const bool query_keep = token_keep && doc >= 0;
    int64_t cb = 0, ce = 0, db = 0, de = 0;
    if (query_keep) {
      int64_t lower = 0;
      if (a.ctx_window > 0) lower = max(lower, anchor - a.ctx_window);
      if (a.q_window > 0) lower = max(lower, anchor + o - a.q_window + 1);
      cb = lower_bound(a.ctx_pos, a.T, lower);
      ce = lower_bound(a.ctx_pos, a.T, anchor);
      const int64_t sd = sortable_doc(doc);
      cb = max(cb, doc_bound(a.ctx_docs, a.T, sd, false));
      ce = min(ce, doc_bound(a.ctx_docs, a.T, sd, true));
      cb = min(cb, ce);
      const int64_t j = lower_bound(a.local_blocks, a.nlb, r);
      if (j < a.nlb && a.local_blocks[j] == r) {
        const int64_t base = a.T + j * a.block;
        int64_t valid = a.block;
        if (a.seq_len > 0) valid = min(max(a.seq_len - anchor, (int64_t)0), a.block);
        db = base;
        de = base + valid;
        if (a.causal) de = min(de, base + o + 1);
        if (a.q_window > 0) {
          db = base + max(o - a.q_window + 1, (int64_t)0);
          de = min(de, base + min(o + a.q_window, a.block));
        }
        db = min(db, de);
      } else {
        db = de = K;
      }
      const int64_t key0 = b * K;
      cb += key0;
      ce += key0;
      db += key0;
      de += key0;
    }
    a.ends[0 * NQ + b * nq + q] = 0;
    a.ends[1 * NQ + b * nq + q] = static_cast<int32_t>(cb);
    a.ends[2 * NQ + b * nq + q] = static_cast<int32_t>(ce);
    a.ends[3 * NQ + b * nq + q] = static_cast<int32_t>(db);
    a.ends[4 * NQ + b * nq + q] = static_cast<int32_t>(de);
  } else if (tid < nq + a.T) {
    const int64_t t = tid - nq;
    if (t > 0) {
      int bad = 0;
      if (a.ctx_pos[t] < a.ctx_pos[t - 1]) bad |= 1;
      if (sortable_doc(a.ctx_docs[t]) < sortable_doc(a.ctx_docs[t - 1])) bad |= 2;
      if (bad) atomicOr(a.flags, bad);
    }
  } else if (tid < nq + a.T + a.nlb && b == 0) {
    const int64_t j = tid - nq - a.T;
    if (a.local_blocks[j] < 0 || a.local_blocks[j] >= a.num_blocks ||
        (j > 0 && a.local_blocks[j] <= a.local_blocks[j - 1]))
      atomicOr(a.flags, 4);
  }
}

struct AuxArgs {
  const int32_t* qaux;  // [4][nq]: anchors, keep, blocks, docs
  const int32_t* kaux;  // [4][nk]: docs, positions, blocks, keep
  int64_t nq, nk, T, block, ctx_window, q_window;
  int causal;
  int32_t* ends;
  int32_t* flags;
};

__device__ __forceinline__ int64_t lower_bound_i32(const int32_t* a, int64_t n, int64_t v) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (a[mid] < v) lo = mid + 1; else hi = mid;
  }
  return lo;
}

__device__ __forceinline__ int64_t doc_bound_i32(const int32_t* docs, int64_t n, int64_t v, bool upper) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    int64_t x = sortable_doc(docs[mid]);
    bool go_right = upper ? (x <= v) : (x < v);
    if (go_right) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Interval endpoints recovered from the eight THD mask tensors (the contract produced by
// thd_attention.py:25-56 at CP=1: context keys first, then each block's B draft keys in order).
// Visibility follows the mask_mod of thd_attention.py:77-131 / _classify_tiles
// (thd_sparse_metadata.py:20-94). Layout assumptions that make the visible set two intervals
// (monotone context positions and documents, kept draft offsets forming a prefix) are checked and
// reported in *flags (bit 1 positions, bit 2 documents, bit 4 draft keep pattern).
__global__ void aux_endpoints_kernel(AuxArgs a) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int32_t* kdocs = a.kaux;
  const int32_t* kpos = a.kaux + a.nk;
  const int32_t* kkeep = a.kaux + 3 * a.nk;
  if (tid < a.nq) {
    const int64_t q = tid;
    const int64_t anchor = a.qaux[q];
    const bool keep = a.qaux[a.nq + q] > 0;
    const int64_t blk = a.qaux[2 * a.nq + q];
    const int64_t doc = a.qaux[3 * a.nq + q];
    const int64_t o = q % a.block;
    int64_t cb = 0, ce = 0, db = 0, de = 0;
    if (keep) {
      int64_t lower = 0;
      if (a.ctx_window > 0) lower = max(lower, anchor - a.ctx_window);
      if (a.q_window > 0) lower = max(lower, anchor + o - a.q_window + 1);
      cb = lower_bound_i32(kpos, a.T, lower);
      ce = lower_bound_i32(kpos, a.T, anchor);
      const int64_t sd = sortable_doc(doc);
      cb = max(cb, doc_bound_i32(kdocs, a.T, sd, false));
      ce = min(ce, doc_bound_i32(kdocs, a.T, sd, true));
      if (doc < 0) ce = cb;  // padding context keys are never kept
      cb = min(cb, ce);
      const int64_t base = a.T + blk * a.block;
      int64_t lo = 0, hi = a.block;
      if (a.causal) hi = min(hi, o + 1);
      if (a.q_window > 0) {
        lo = max(lo, o - a.q_window + 1);
        hi = min(hi, o + a.q_window);
      }
      // kept draft offsets of this block: a prefix [0, kept)
      int64_t kept = 0;
      if (base >= a.T && base + a.block <= a.nk) {
        while (kept < a.block && kkeep[base + kept] > 0 && kdocs[base + kept] == doc) ++kept;
        for (int64_t j = kept; j < a.block; ++j)
          if (kkeep[base + j] > 0 && kdocs[base + j] == doc) { atomicOr(a.flags, 4); break; }
      }
      hi = min(hi, kept);
      lo = min(lo, hi);
      db = base + lo;
      de = base + hi;
    }
    a.ends[q] = 0;
    a.ends[1 * a.nq + q] = static_cast<int32_t>(cb);
    a.ends[2 * a.nq + q] = static_cast<int32_t>(ce);
    a.ends[3 * a.nq + q] = static_cast<int32_t>(db);
    a.ends[4 * a.nq + q] = static_cast<int32_t>(de);
  } else if (tid < a.nq + a.T && tid > a.nq) {
    const int64_t t = tid - a.nq;
    int bad = 0;
    if (kpos[t] < kpos[t - 1]) bad |= 1;
    if (sortable_doc(kdocs[t]) < sortable_doc(kdocs[t - 1])) bad |= 2;
    if (bad) atomicOr(a.flags, bad);
  }
}

struct TileArgs {
  const int32_t* ends;
  int64_t nq, nk, tm, tn, nm, nn;
  int pad_visible;
  int32_t* classes;
  int32_t* pcnt;
  int32_t* pidx;
  int32_t* fcnt;
  int32_t* fidx;
};

constexpr int kTileThreads = 256;
constexpr int kMaxStagedRows = 1024;

__device__ __forceinline__ int64_t overlap(int64_t a0, int64_t a1, int64_t b0, int64_t b1) {
  return max(min(a1, b1) - max(a0, b0), (int64_t)0);
}

// One workgroup per query tile m: classify every key tile of the row, then compact the row into
// the ordered partial / full lists with a wave ballot scan.
__global__ void __launch_bounds__(kTileThreads) classify_rows_kernel(TileArgs a) {
  __shared__ int32_t s_ends[4][kMaxStagedRows];
  const int64_t m = blockIdx.x;
  const int64_t r0 = m * a.tm;
  const int64_t r1 = min(r0 + a.tm, a.nq);
  const int rows = static_cast<int>(r1 - r0);
  for (int i = threadIdx.x; i < rows; i += blockDim.x) {
    s_ends[0][i] = a.ends[1 * a.nq + r0 + i];
    s_ends[1][i] = a.ends[2 * a.nq + r0 + i];
    s_ends[2][i] = a.ends[3 * a.nq + r0 + i];
    s_ends[3][i] = a.ends[4 * a.nq + r0 + i];
  }
  __syncthreads();
  int32_t* cls_row = a.classes + m * a.nn;
  const bool rows_padded = r0 + a.tm > a.nq;
  for (int64_t n = threadIdx.x; n < a.nn; n += blockDim.x) {
    const int64_t k0 = n * a.tn;
    const int64_t k1 = min(k0 + a.tn, a.nk);
    const int64_t width = k1 - k0;
    bool any = false, all = true;
    for (int i = 0; i < rows; ++i) {
      const int64_t c = overlap(k0, k1, s_ends[0][i], s_ends[1][i]) +
                        overlap(k0, k1, s_ends[2][i], s_ends[3][i]);
      any |= c > 0;
      all &= c == width;
    }
    if (!a.pad_visible && (rows_padded || k0 + a.tn > a.nk)) all = false;
    cls_row[n] = any ? (all ? 2 : 1) : 0;
  }
  __syncthreads();
  if (threadIdx.x < kWave && (a.pidx || a.fidx || a.pcnt || a.fcnt)) {
    const int lane = threadIdx.x;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int pc = 0, fc = 0;
    int32_t* prow = a.pidx ? a.pidx + m * a.nn : nullptr;
    int32_t* frow = a.fidx ? a.fidx + m * a.nn : nullptr;
    for (int64_t n0 = 0; n0 < a.nn; n0 += kWave) {
      const int64_t n = n0 + lane;
      const int cls = n < a.nn ? cls_row[n] : 0;
      const uint64_t pm = __ballot(cls == 1);
      const uint64_t fm = __ballot(cls == 2);
      if (cls == 1 && prow) prow[pc + __popcll(pm & below)] = static_cast<int32_t>(n);
      if (cls == 2 && frow) frow[fc + __popcll(fm & below)] = static_cast<int32_t>(n);
      pc += __popcll(pm);
      fc += __popcll(fm);
    }
    if (prow) for (int64_t n = pc + lane; n < a.nn; n += kWave) prow[n] = 0;
    if (frow) for (int64_t n = fc + lane; n < a.nn; n += kWave) frow[n] = 0;
    if (lane == 0) {
      if (a.pcnt) a.pcnt[m] = pc;
      if (a.fcnt) a.fcnt[m] = fc;
    }
  }
}

// One wave per key tile n: ordered lists of the query tiles that see it (the transpose).
__global__ void __launch_bounds__(kWave) compact_columns_kernel(TileArgs a) {
  const int64_t n = blockIdx.x;
  const int lane = threadIdx.x;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int pc = 0, fc = 0;
  int32_t* prow = a.pidx ? a.pidx + n * a.nm : nullptr;
  int32_t* frow = a.fidx ? a.fidx + n * a.nm : nullptr;
  for (int64_t m0 = 0; m0 < a.nm; m0 += kWave) {
    const int64_t m = m0 + lane;
    const int cls = m < a.nm ? a.classes[m * a.nn + n] : 0;
    const uint64_t pm = __ballot(cls == 1);
    const uint64_t fm = __ballot(cls == 2);
    if (cls == 1 && prow) prow[pc + __popcll(pm & below)] = static_cast<int32_t>(m);
    if (cls == 2 && frow) frow[fc + __popcll(fm & below)] = static_cast<int32_t>(m);
    pc += __popcll(pm);
    fc += __popcll(fm);
  }
  if (prow) for (int64_t m = pc + lane; m < a.nm; m += kWave) prow[m] = 0;
  if (frow) for (int64_t m = fc + lane; m < a.nm; m += kWave) frow[m] = 0;
  if (lane == 0) {
    if (a.pcnt) a.pcnt[n] = pc;
    if (a.fcnt) a.fcnt[n] = fc;
  }
}

}  // namespace

int launch_tile_metadata(const int32_t* ends, int64_t nq, int64_t nk, int64_t tm, int64_t tn,
                         int pad_visible, int32_t* classes, int32_t* fpc, int32_t* fpi,
                         int32_t* ffc, int32_t* ffi, int32_t* bpc, int32_t* bpi, int32_t* bfc,
                         int32_t* bfi, hipStream_t stream) {
  TileArgs a;
  a.ends = ends;
  a.nq = nq;
  a.nk = nk;
  a.tm = tm;
  a.tn = tn;
  a.nm = (nq + tm - 1) / tm;
  a.nn = (nk + tn - 1) / tn;
  a.pad_visible = pad_visible;
  a.classes = classes;
  a.pcnt = fpc;
  a.pidx = fpi;
  a.fcnt = ffc;
  a.fidx = ffi;
  hipLaunchKernelGGL(classify_rows_kernel, dim3(static_cast<uint32_t>(a.nm)), dim3(kTileThreads), 0,
                     stream, a);
  int rc = check_launch("classify_rows_kernel");
  if (rc) return rc;
  if (bpc || bpi || bfc || bfi) {
    a.pcnt = bpc;
    a.pidx = bpi;
    a.fcnt = bfc;
    a.fidx = bfi;
    hipLaunchKernelGGL(compact_columns_kernel, dim3(static_cast<uint32_t>(a.nn)), dim3(kWave), 0,
                       stream, a);
    rc = check_launch("compact_columns_kernel");
  }
  return rc;
}

}  // namespace aspec

using namespace aspec;

extern "C" int aspec_thd_batch_row_metadata(const int64_t* anchors, const uint8_t* keep,
                                            const int64_t* anchor_docs,
                                            const int64_t* context_positions,
                                            const int64_t* context_docs, int64_t batch,
                                            int64_t num_blocks, int64_t block_size,
                                            int64_t context_length, int64_t sequence_length,
                                            int64_t context_window, int64_t query_window,
                                            int draft_is_causal, int32_t* query_aux,
                                            int32_t* key_aux, int32_t* endpoints,
                                            int32_t* status_flags, void* stream) {
  if (batch <= 0 || batch > 65535 || num_blocks < 0 || block_size <= 0 || context_length < 0)
    return set_error(ASPEC_ERR_INVALID,
                     "invalid THD geometry (batch=%lld, blocks=%lld, block=%lld, T=%lld)",
                     (long long)batch, (long long)num_blocks, (long long)block_size,
                     (long long)context_length);
  const int64_t nq = num_blocks * block_size;
  const int64_t K = context_length + nq;
  if (batch * K >= (1LL << 31) - 1)
    return set_error(ASPEC_ERR_INVALID, "THD metadata exceeds int32 indexing (%lld keys)",
                     (long long)(batch * K));
  if (num_blocks > 0 && (!anchors || !keep || !anchor_docs))
    return set_error(ASPEC_ERR_INVALID, "anchors, keep and anchor_docs are required");
  if (context_length > 0 && (!context_positions || !context_docs))
    return set_error(ASPEC_ERR_INVALID, "context positions and document ids are required");
  const int64_t total = nq + context_length;
  if (total == 0) return ASPEC_OK;
  RowArgs a;
  a.anchors = anchors;
  a.keep = keep;
  a.anchor_docs = anchor_docs;
  a.ctx_pos = context_positions;
  a.ctx_docs = context_docs;
  a.num_blocks = num_blocks;
  a.block = block_size;
  a.T = context_length;
  a.seq_len = sequence_length;
  a.ctx_window = context_window;
  a.q_window = query_window;
  a.causal = draft_is_causal;
  a.qaux = query_aux;
  a.kaux = key_aux;
  a.ends = endpoints;
  a.flags = status_flags;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(row_metadata_kernel,
                     dim3(static_cast<uint32_t>(blocks), static_cast<uint32_t>(batch)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("row_metadata_kernel");
}

extern "C" int aspec_thd_cp_shard_endpoints(const int64_t* anchors, const uint8_t* keep,
                                            const int64_t* anchor_docs,
                                            const int64_t* context_positions,
                                            const int64_t* context_docs, int64_t batch,
                                            int64_t num_blocks, int64_t block_size,
                                            int64_t context_length, const int64_t* query_blocks,
                                            int64_t num_query_blocks, const int64_t* local_blocks,
                                            int64_t num_local_blocks, int64_t sequence_length,
                                            int64_t context_window, int64_t query_window,
                                            int draft_is_causal, int32_t* endpoints,
                                            int32_t* status_flags, void* stream) {
  if (batch <= 0 || batch > 65535 || num_blocks < 0 || block_size <= 0 || context_length < 0 ||
      num_query_blocks < 0 || num_local_blocks < 0 || num_local_blocks > num_blocks)
    return set_error(ASPEC_ERR_INVALID,
                     "invalid CP shard geometry (batch=%lld, blocks=%lld, query blocks=%lld, "
                     "local blocks=%lld, block=%lld, T=%lld)",
                     (long long)batch, (long long)num_blocks, (long long)num_query_blocks,
                     (long long)num_local_blocks, (long long)block_size, (long long)context_length);
  const int64_t nq = num_query_blocks * block_size;
  const int64_t K = context_length + num_local_blocks * block_size;
  if (batch * K >= (1LL << 31) - 1 || batch * nq >= (1LL << 31) - 1)
    return set_error(ASPEC_ERR_INVALID, "CP shard metadata exceeds int32 indexing (%lld keys)",
                     (long long)(batch * K));
  if (!endpoints || !status_flags)
    return set_error(ASPEC_ERR_INVALID, "endpoints and status flags are required");
  if (num_blocks > 0 && (!anchors || !keep || !anchor_docs))
    return set_error(ASPEC_ERR_INVALID, "anchors, keep and anchor_docs are required");
  if ((num_query_blocks > 0 && !query_blocks) || (num_local_blocks > 0 && !local_blocks))
    return set_error(ASPEC_ERR_INVALID, "query and local block ids are required");
  if (context_length > 0 && (!context_positions || !context_docs))
    return set_error(ASPEC_ERR_INVALID, "context positions and document ids are required");
  const int64_t total = nq + context_length + num_local_blocks;
  if (total == 0) return ASPEC_OK;
  ShardArgs a;
  a.anchors = anchors;
  a.keep = keep;
  a.anchor_docs = anchor_docs;
  a.ctx_pos = context_positions;
  a.ctx_docs = context_docs;
  a.query_blocks = query_blocks;
  a.local_blocks = local_blocks;
  a.num_blocks = num_blocks;
  a.nqb = num_query_blocks;
  a.nlb = num_local_blocks;
  a.block = block_size;
  a.T = context_length;
  a.seq_len = sequence_length;
  a.ctx_window = context_window;
  a.q_window = query_window;
  a.causal = draft_is_causal;
  a.ends = endpoints;
  a.flags = status_flags;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(shard_endpoints_kernel,
                     dim3(static_cast<uint32_t>(blocks), static_cast<uint32_t>(batch)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("shard_endpoints_kernel");
}

extern "C" int aspec_thd_row_metadata(const int64_t* anchors, const uint8_t* keep,
                                      const int64_t* anchor_docs, const int64_t* context_positions,
                                      const int64_t* context_docs, int64_t num_blocks,
                                      int64_t block_size, int64_t context_length,
                                      int64_t sequence_length, int64_t context_window,
                                      int64_t query_window, int draft_is_causal,
                                      int32_t* query_aux, int32_t* key_aux, int32_t* endpoints,
                                      int32_t* status_flags, void* stream) {
  return aspec_thd_batch_row_metadata(anchors, keep, anchor_docs, context_positions, context_docs,
                                      1, num_blocks, block_size, context_length, sequence_length,
                                      context_window, query_window, draft_is_causal, query_aux,
                                      key_aux, endpoints, status_flags, stream);
}

extern "C" int aspec_thd_aux_endpoints(const int32_t* query_aux, const int32_t* key_aux,
                                       int64_t num_queries, int64_t num_keys, int64_t block_size,
                                       int64_t context_window, int64_t query_window,
                                       int draft_is_causal, int32_t* endpoints,
                                       int32_t* status_flags, void* stream) {
  if (num_queries <= 0 || num_keys < num_queries || block_size <= 0)
    return set_error(ASPEC_ERR_INVALID, "Invalid THD fixed sparse geometry");
  if (!query_aux || !key_aux || !endpoints || !status_flags)
    return set_error(ASPEC_ERR_INVALID, "Expected eight THD fixed mask tensors");
  AuxArgs a;
  a.qaux = query_aux;
  a.kaux = key_aux;
  a.nq = num_queries;
  a.nk = num_keys;
  a.T = num_keys - num_queries;
  a.block = block_size;
  a.ctx_window = context_window;
  a.q_window = query_window;
  a.causal = draft_is_causal;
  a.ends = endpoints;
  a.flags = status_flags;
  const int64_t total = num_queries + a.T;
  const int threads = 256;
  hipLaunchKernelGGL(aux_endpoints_kernel, dim3(static_cast<uint32_t>((total + threads - 1) / threads)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("aux_endpoints_kernel");
}

extern "C" int aspec_thd_tile_metadata(const int32_t* endpoints, int64_t num_queries,
                                       int64_t num_keys, int64_t tile_m, int64_t tile_n,
                                       int pad_visible, int32_t* classes, int32_t* fwd_partial_cnt,
                                       int32_t* fwd_partial_idx, int32_t* fwd_full_cnt,
                                       int32_t* fwd_full_idx, int32_t* bwd_partial_cnt,
                                       int32_t* bwd_partial_idx, int32_t* bwd_full_cnt,
                                       int32_t* bwd_full_idx, void* stream) {
  if (num_queries <= 0 || num_keys <= 0 || tile_m <= 0 || tile_n <= 0)
    return set_error(ASPEC_ERR_INVALID, "Invalid THD fixed sparse geometry");
  if (tile_m > kMaxStagedRows)
    return set_error(ASPEC_ERR_UNSUPPORTED, "tile_m %lld exceeds %d", (long long)tile_m, kMaxStagedRows);
  if (!endpoints || !classes)
    return set_error(ASPEC_ERR_INVALID, "endpoints and classes buffers are required");
  return launch_tile_metadata(endpoints, num_queries, num_keys, tile_m, tile_n, pad_visible, classes,
                              fwd_partial_cnt, fwd_partial_idx, fwd_full_cnt, fwd_full_idx,
                              bwd_partial_cnt, bwd_partial_idx, bwd_full_cnt, bwd_full_idx,
                              static_cast<hipStream_t>(stream));
}
