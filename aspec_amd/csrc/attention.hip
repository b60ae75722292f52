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
// Tile loops are software pipelined: the next tile streams from global memory straight into LDS
// while the current one is computed.
#include "attn_common.h"
#include "plan.h"

namespace aspec {
namespace {

constexpr int kTM = kFwdTileM;          // query rows per wave (one per lane column)
constexpr int kTN = kFwdTileN;          // keys per tile
constexpr int kMaxGroup = 8;
constexpr int kKvWaves = kBwdTileN / 32;
// Online softmax keeps a stale row maximum until a tile raises it by more than 2^8: exp2 of the
// shifted scores stays <= 256 (exact in fp32, fine in bf16) and O is rescaled only then.
constexpr float kRescaleThreshold = 8.f;
// LDS read-ahead (k-steps) of the score chains of the forward and dQ kernels.
constexpr int kFwdAhead = 1;
constexpr int kDqAhead = 1;

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
  float* ws_dk;        // [kMaxChunks][K][Hkv][D] fp32 partials of key tiles split over units
  float* ws_dv;
  uint16_t* dq; int64_t dqst, dqsh;
  uint16_t* dk; int64_t dkst, dksh;
  uint16_t* dv; int64_t dvst, dvsh;
};

// A row-major operand in a swizzled LDS tile: this lane's row at `off` (row_operand_off), read
// one 16-dim k-step at a time.
struct RowOperand {
  const uint16_t* tile;
  int off;
  __device__ __forceinline__ uint4 step(int ds) const { return load16(tile + (off ^ (ds << 4))); }
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

// The MFMA chains below load their LDS operands a few k-steps ahead and fence each step with a
// scheduling barrier: without it the scheduler hoists every LDS read of the tile to the top,
// which overflows the VGPR budget and parks operands in AGPRs.
#define ASPEC_STEP_FENCE() __builtin_amdgcn_sched_barrier(0)

// Two independent 8-step chains: acc0 = A0 x B0, acc1 = A1 x B1 over the 128-dim reduction. A rows
// live in LDS (`ra0` / `ra1`), read AHEAD k-steps ahead of their MFMA; the B operands come from
// registers.
template <int AHEAD, bool F16 = false, typename Operand>
__device__ __forceinline__ void mfma_chains2(f32x16& acc0, f32x16& acc1, const Operand& ra0,
                                             const Operand& ra1, const bf16x8 (&b0)[8],
                                             const bf16x8 (&b1)[8]) {
  acc0 = f32x16{};
  acc1 = f32x16{};
  uint4 x0[8], x1[8];
#pragma unroll
  for (int ds = 0; ds < AHEAD; ++ds) {
    x0[ds] = ra0.step(ds);
    x1[ds] = ra1.step(ds);
  }
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) {
    if (ds + AHEAD < 8) {
      x0[ds + AHEAD] = ra0.step(ds + AHEAD);
      x1[ds + AHEAD] = ra1.step(ds + AHEAD);
    }
    acc0 = mfma32<F16>(as_bf16x8(x0[ds]), b0[ds], acc0);
    acc1 = mfma32<F16>(as_bf16x8(x1[ds]), b1[ds], acc1);
    ASPEC_STEP_FENCE();
  }
}

// Per-lane LDS byte offsets of a wave's reads of one 64 x 128 K/V tile, computed once per kernel:
// the row reads of k-step ds (`row`) and the transposed reads of column block d (`tr`, the two
// halves). Everything else in those addresses (the stage, the 32-row half, the k-step row block)
// is a compile-time constant that lands in the instructions' offset field, so the tile loop spends
// no VALU on LDS addresses.
struct TileOffsets {
  uint32_t row[8];
  uint32_t tr[4][2];
  __device__ __forceinline__ explicit TileOffsets(int lane) {
    const int ro = row_operand_off(lane & 31, lane >> 5);
    const TrOffsets t(lane);
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) row[ds] = static_cast<uint32_t>(ro ^ (ds << 4)) * 2u;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      tr[d][0] = static_cast<uint32_t>(t.lo ^ (d * 32)) * 2u;
      tr[d][1] = static_cast<uint32_t>(t.hi ^ (d * 32)) * 2u;
    }
  }
};

// A wave-uniform value behind an empty asm: the compiler keeps it in SGPRs as computed and cannot
// rematerialize it (for instance by reloading a kernel argument inside a loop).
template <typename T>
__device__ __forceinline__ T opaque_s(T x) {
  asm volatile("" : "+s"(x));
  return x;
}

__device__ __forceinline__ const char* byte_ptr(const uint16_t* p) { return reinterpret_cast<const char*>(p); }

// The row-read half of TileOffsets alone, for kernels without register room for the other half.
struct RowOffsets {
  uint32_t row[8];
  __device__ __forceinline__ explicit RowOffsets(int lane) {
    const int ro = row_operand_off(lane & 31, lane >> 5);
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) row[ds] = static_cast<uint32_t>(ro ^ (ds << 4)) * 2u;
  }
};

struct RowOperandR {
  const uint16_t* tile;
  const RowOffsets& o;
  __device__ __forceinline__ uint4 step(int ds) const {
    return *reinterpret_cast<const uint4*>(byte_ptr(tile) + o.row[ds]);
  }
};

// Row-major operand read through TileOffsets.
struct RowOperandT {
  const uint16_t* tile;
  const TileOffsets& o;
  __device__ __forceinline__ uint4 step(int ds) const {
    return *reinterpret_cast<const uint4*>(byte_ptr(tile) + o.row[ds]);
  }
};

// Transposed fragment (rows ks*16 .. +15, columns d*32 .. +31) read through TileOffsets.
__device__ __forceinline__ bf16x8 read_tr_t(const uint16_t* tile, const TileOffsets& o, int ks, int d) {
  const char* b = byte_ptr(tile) + ks * 16 * kRowLd * 2;
  const s16x4 lo = ds_read_tr16(reinterpret_cast<const uint16_t*>(b + o.tr[d][0]));
  const s16x4 hi = ds_read_tr16(reinterpret_cast<const uint16_t*>(b + o.tr[d][1]));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
  const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
  return as_bf16x8(uint4{l2.x, l2.y, h2.x, h2.y});
}

// acc[d] += A(d, ks) x B[ks] as mfma_tr_blocks, with the fragments read through TileOffsets;
// `cur` holds k-step 0.
template <int KS, bool F16 = false>
__device__ __forceinline__ void mfma_tr_blocks_t(f32x16 (&acc)[4], const uint16_t* tile,
                                                 const TileOffsets& o, bf16x8 (&cur)[4],
                                                 const bf16x8 (&b)[KS]) {
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    bf16x8 nxt[4];
    if (ks + 1 < KS) {
#pragma unroll
      for (int d = 0; d < 4; ++d) nxt[d] = read_tr_t(tile, o, ks + 1, d);
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) acc[d] = mfma32<F16>(cur[d], b[ks], acc[d]);
    ASPEC_STEP_FENCE();
    if (ks + 1 < KS) {
#pragma unroll
      for (int d = 0; d < 4; ++d) cur[d] = nxt[d];
    }
  }
}

// Sum of the 32 values of four packed operands (the rounded P that the P.V MFMAs use), two at a
// time with the bf16 (fp16) dot product against ones.
template <bool F16 = false>
__device__ __forceinline__ float sum_p(const bf16x8 (&pb)[4]) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2v;
  float acc0 = 0.f, acc1 = 0.f;
  auto dot = [](uint32_t w, float acc) __attribute__((always_inline)) {
    if constexpr (F16) {
      const f16x2_t ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
      return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), ones, acc, false);
    } else {
      const bf16x2v ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
      return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, w), ones, acc, false);
    }
  };
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 v = __builtin_bit_cast(uint4, pb[i]);
    acc0 = dot(v.x, acc0);
    acc1 = dot(v.y, acc1);
    acc0 = dot(v.z, acc0);
    acc1 = dot(v.w, acc1);
  }
  return acc0 + acc1;
}

// First k-step fragments of mfma_tr_blocks, read early so that their latency hides under the
// caller's softmax work.
__device__ __forceinline__ void read_tr_first(bf16x8 (&cur)[4], const uint16_t* tile, const TrOffsets& tro) {
#pragma unroll
  for (int d = 0; d < 4; ++d) cur[d] = read_tr_operand(tile, tro, 0, d * 32);
}

// acc[d] += A(d, ks) x B[ks] for d = 0..3 and k-steps ks = 0..KS-1, where A(d, ks) is the
// transposed fragment of the row-major LDS `tile` (rows = the reduction index, 16 per k-step;
// columns d*32 .. +32 = the output rows), read with transpose loads; `cur` holds k-step 0
// (read_tr_first).
template <int KS, bool F16 = false>
__device__ __forceinline__ void mfma_tr_blocks(f32x16 (&acc)[4], const uint16_t* tile,
                                               const TrOffsets& tro, bf16x8 (&cur)[4],
                                               const bf16x8 (&b)[KS]) {
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    bf16x8 nxt[4];
    if (ks + 1 < KS) {
#pragma unroll
      for (int d = 0; d < 4; ++d) nxt[d] = read_tr_operand(tile, tro, (ks + 1) * 16, d * 32);
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) acc[d] = mfma32<F16>(cur[d], b[ks], acc[d]);
    ASPEC_STEP_FENCE();
    if (ks + 1 < KS) {
#pragma unroll
      for (int d = 0; d < 4; ++d) cur[d] = nxt[d];
    }
  }
}

template <bool F16 = false>
__device__ __forceinline__ void store_row_c(uint16_t* dst, const f32x16 (&acc)[4], float mul, int g) {
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      u32x2 w;
      w.x = pack_elem2<F16>(acc[db][rq * 4 + 0] * mul, acc[db][rq * 4 + 1] * mul);
      w.y = pack_elem2<F16>(acc[db][rq * 4 + 2] * mul, acc[db][rq * 4 + 3] * mul);
      *reinterpret_cast<u32x2*>(dst + db * 32 + rq * 8 + g * 4) = w;
    }
  }
}

// Direct global -> LDS loads (gfx950 global_load_lds_dword / _dwordx4): lane l's bytes land at
// `lds_wave_base` + l * size; the base, which goes through M0, must be the same for the whole
// wave. They are issued from inline assembly so the compiler's wait-count bookkeeping never sees
// them: it would otherwise wait for every one of them before each LDS read and barrier, which
// defeats loading two iterations ahead. Callers wait for them explicitly (vmcnt). The compiler's
// own vector loads are issued before or after these and return in order, so its waits stay
// correct (at worst they also cover these loads). M0 is written one instruction before its use.
// The LDS byte address of a pointer into __shared__ memory: the low 32 bits of its flat address
// (the shared aperture occupies the high half). Taken without an address-space cast, whose null
// check the compiler can otherwise lower into an illegal compare against src_shared_base.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}
// 16 bytes per lane, addressed as a wave-uniform 64-bit base (SGPRs) plus a 32-bit per-lane byte
// offset.
__device__ __forceinline__ void lds_load16_at(const void* base, uint32_t byte_off, void* lds_wave_base) {
  // readfirstlane returns int: go through uint32_t so the low word is zero-extended, not
  // sign-extended into the high word.
  const uint64_t b = reinterpret_cast<uintptr_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint64_t sbase = static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_address(lds_wave_base)), "v"(byte_off), "s"(sbase)
               : "memory", "m0");
}
// Same with 4 bytes per lane.
__device__ __forceinline__ void lds_load4_at(const void* base, uint32_t byte_off, void* lds_wave_base) {
  const uint64_t b = reinterpret_cast<uintptr_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint64_t sbase = static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(lds_address(lds_wave_base)), "v"(byte_off), "s"(sbase)
               : "memory", "m0");
}


// K/V tile ring of the query-major kernels (forward, dQ): two stages, each a 64-key K tile and V
// tile in swizzled rows, filled straight from global memory (no staging registers). Stage t+1 is
// loading while stage t is computed; one wait and one barrier per tile.
struct KvStageFwd {
  uint16_t k[kTN * kRowLd];
  uint16_t v[kTN * kRowLd];
};

// Issues this wave's share of the loads of the key tile at key0 into `st`: 32 wave-wide loads of
// four rows each (16 for K, 16 for V), wave w taking loads w, w+G, ... Load i fills physical rows
// 4(i%16) + l/16 (lane l at physical chunk l%16), so lane l fetches the logical chunk stored
// there: (l%16) ^ swz(row). With row % 16 = 4q + s (q = i%4, s = l/16), swz(row) = swz(s) ^ T(q),
// T(q) = (q&1) | (q&2)<<2, so the per-lane part `lane_chunk` = (l%16 ^ swz(s)) * 16 bytes is fixed
// and each load costs one xor with a wave-uniform value. The tile base lives in SGPRs and the
// per-lane offset is 32-bit (rows x stride < 2^31 is checked on the host). Keys past the tensor
// repeat its last row (such tiles are always partial: the mask drops them).
struct KvTileLanes {
  uint32_t lane_chunk;  // (l%16 ^ swz(l/16)) * 16
  int rsub;             // l / 16
  __device__ __forceinline__ explicit KvTileLanes(int lane)
      : lane_chunk(static_cast<uint32_t>(((lane & 15) ^ swz(lane >> 4)) << 4)), rsub(lane >> 4) {}
};

template <int G>
__device__ __forceinline__ void issue_kv_tile(const uint16_t* kbase, int64_t kst,
                                              const uint16_t* vbase, int64_t vst, int key0,
                                              int nk, KvStageFwd& st, int wave,
                                              const KvTileLanes& ln) {
  const uint16_t* ktile = kbase + static_cast<int64_t>(key0) * kst;
  const uint16_t* vtile = vbase + static_cast<int64_t>(key0) * vst;
  const int last = min(nk - 1 - key0, kTN - 1);  // rows past it repeat it
  const uint32_t kst2 = static_cast<uint32_t>(kst * 2), vst2 = static_cast<uint32_t>(vst * 2);
#pragma unroll
  for (int p = 0; p < (32 + G - 1) / G; ++p) {
    const int i = wave + p * G;
    if (i >= 32) break;
    const int q = i & 3;
    const uint32_t chunk = ln.lane_chunk ^ static_cast<uint32_t>(((q & 1) | ((q & 2) << 2)) << 4);
    const int row = min((i & 15) * 4 + ln.rsub, last);
    const uint32_t off = static_cast<uint32_t>(row) * (i < 16 ? kst2 : vst2) + chunk;
    uint16_t* dst = (i < 16 ? st.k : st.v) + (i & 15) * 4 * kRowLd;
    lds_load16_at(i < 16 ? ktile : vtile, off, dst);
  }
}

// The plan list of one query tile, 64 entries at a time in one VGPR (lane j: entry base + j), read
// with readlane: no memory access (and so no wait on the in-flight tile loads) inside the loop.
struct ListWindow {
  const int32_t* list;
  int count, base, reg;
  __device__ __forceinline__ void load(int b, int lane) {
    base = b;
    reg = b + lane < count ? list[b + lane] : 0;
  }
  __device__ __forceinline__ uint32_t entry(int t) const {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(reg, t - base));
  }
};

// ---------------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------------
// Online softmax of one 64-key tile of scores S^T (`s`, lane = query row): masks a partial tile,
// raises the running maximum (rescaling O and the row sum only when it grows by more than
// kRescaleThreshold), and leaves P, rounded to bf16, in `pb` as the P.V operand.
template <bool F16>
__device__ __forceinline__ void fwd_softmax(f32x16 (&s)[2], f32x16 (&oacc)[4], float& m_run,
                                            float& l_run, bool partial, const RowIntervals& iv,
                                            float scale_log2, int g, bf16x8 (&pb)[4]) {
  // Row maximum of the raw scores (scale > 0 commutes with max); the scale then folds into the
  // exponent: p = exp2(s * scale*log2e - m).
  if (partial) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = masked_score(s[kb][r], iv.word(kb, g), r);
  }
  float tile_max = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) tile_max = fmaxf(tile_max, s[kb][r]);
  }
  tile_max = max_halves(tile_max) * scale_log2;
  const bool grow = tile_max > m_run + kRescaleThreshold;
  if (__any(grow)) {
    const float m_new = grow ? tile_max : m_run;
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < 4; ++d) oacc[d] *= alpha;
  }
  const float neg_m = -m_run;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kb][r] = fast_exp2(fmaf(s[kb][r], scale_log2, neg_m));
  }
  pb[0] = pack_c_half<F16>(s[0], 0);
  pb[1] = pack_c_half<F16>(s[0], 8);
  pb[2] = pack_c_half<F16>(s[1], 0);
  pb[3] = pack_c_half<F16>(s[1], 8);
  // The row sum is taken over the rounded P that the P.V product uses, so O is normalized by
  // exactly the weights it was built from.
  l_run += sum_p<F16>(pb);
}

template <bool F16>
__device__ __forceinline__ void fwd_tile(const uint16_t* sk, const uint16_t* sv,
                                         const bf16x8 (&qf)[8], f32x16 (&oacc)[4], float& m_run,
                                         float& l_run, bool partial, const RowIntervals& iv, float scale_log2,
                                         const TileOffsets& o, int g) {
  f32x16 s[2];
  mfma_chains2<kFwdAhead, F16>(s[0], s[1], RowOperandT{sk, o}, RowOperandT{sk + 32 * kRowLd, o}, qf, qf);
  bf16x8 vcur[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) vcur[d] = read_tr_t(sv, o, 0, d);
  bf16x8 pb[4];
  fwd_softmax<F16>(s, oacc, m_run, l_run, partial, iv, scale_log2, g, pb);
  mfma_tr_blocks_t<4, F16>(oacc, sv, o, vcur, pb);
}

// Two K/V stages (64 KB) per workgroup, two workgroups per CU: the next tile streams into LDS
// while this one is computed, and the two workgroups overlap each other's MFMA and softmax work.
template <int G, bool F16>
__device__ __forceinline__ void attn_fwd_body(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) KvStageFwd ring[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wave >= 0 && wave < G);
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t m = a.plan.nmf - 1 - blockIdx.x / a.hkv;  // longest prefixes first
  const int head = hkv * G + wave;
  const int64_t qrow = m * kTM + c;
  const bool valid_q = qrow < a.nq;
  const int64_t qsafe = valid_q ? qrow : a.nq - 1;

  const uint16_t* kbase = a.k + hkv * a.ksh;
  const uint16_t* vbase = a.v + hkv * a.vsh;
  const int nk = static_cast<int>(a.nk);
  ListWindow lw{a.plan.f_list + m * a.plan.nnf, a.plan.f_cnt[m], 0, 0};
  lw.load(0, lane);
  const KvTileLanes lanes(lane);
  auto issue = [&](uint32_t entry, KvStageFwd& stage) __attribute__((always_inline)) {
    const int key0 = static_cast<int>(entry & ~kFullBit) * kTN;
    issue_kv_tile<G>(kbase, a.kst, vbase, a.vst, key0, nk, stage, wave, lanes);
  };
  if (lw.count > 0) issue(lw.entry(0), ring[0]);

  bf16x8 qf[8];
  load_row_frag(qf, a.q + qsafe * a.qst + head * a.qsh, valid_q, g);
  int cb = a.ends[1 * a.nq + qsafe], ce = a.ends[2 * a.nq + qsafe];
  int db = a.ends[3 * a.nq + qsafe], de = a.ends[4 * a.nq + qsafe];
  if (!valid_q) cb = ce = db = de = 0;

  f32x16 oacc[4] = {};
  float m_run = kMaskValue;
  float l_run = 0.f;
  const TileOffsets offs(lane);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  lds_barrier();

  // Tile t computes from ring[t % 2] while tile t+1 streams into the other stage; the loop is
  // unrolled by two so that each stage's LDS address is a constant.
  auto tile = [&](int t, const KvStageFwd& cur, KvStageFwd& nxt) __attribute__((always_inline)) {
    const uint32_t entry = lw.entry(t);
    if (t + 1 < lw.count) {
      if (t + 1 - lw.base == kWave) lw.load(t + 1, lane);  // nothing else in flight here
      issue(lw.entry(t + 1), nxt);
    }
    RowIntervals iv;
    iv.at_tile(static_cast<int>((entry & ~kFullBit) * kTN), cb, ce, db, de);
    fwd_tile<F16>(cur.k, cur.v, qf, oacc, m_run, l_run, !(entry & kFullBit), iv, a.scale_log2, offs, g);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's loads of tile t+1 have landed
    lds_barrier();
  };
  for (int t = 0; t < lw.count; t += 2) {
    tile(t, ring[0], ring[1]);
    if (t + 1 >= lw.count) break;
    tile(t + 1, ring[1], ring[0]);
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (valid_q) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    store_row_c<F16>(a.out + qrow * a.ost + head * a.osh, oacc, inv, g);
    if (g == 0) a.lse[static_cast<int64_t>(head) * a.nq + qrow] =
        l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : kMaskValue;
  }
}

// bf16 and fp16 instances (one kernel name per element type).
template <int G>
__global__ void __launch_bounds__(kWave * G, 2) attn_fwd_kernel(AttnArgs a) { attn_fwd_body<G, false>(a); }
template <int G>
__global__ void __launch_bounds__(kWave * G, 2) attn_fwd_f16_kernel(AttnArgs a) { attn_fwd_body<G, true>(a); }

// ---------------------------------------------------------------------------------------------
// Backward prepare: delta = rowsum(dO * O) - dLSE, lse2 = LSE * log2(e) (16 lanes per row).
// ---------------------------------------------------------------------------------------------
template <bool F16>
__device__ __forceinline__ void attn_bwd_pre_body(AttnArgs a) {
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
    for (int e = 0; e < 8; ++e) acc += elem_to_f32<F16>(half_of(o, e)) * elem_to_f32<F16>(half_of(d, e));
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (valid && chunk == 0) {
    const float dl = a.dlse ? a.dlse[row] : 0.f;
    a.ws_delta[row] = acc - dl;
    a.ws_lse2[row] = a.lse_in[row] * kLog2e;
  }
}

__global__ void __launch_bounds__(256) attn_bwd_pre_kernel(AttnArgs a) { attn_bwd_pre_body<false>(a); }
__global__ void __launch_bounds__(256) attn_bwd_pre_f16_kernel(AttnArgs a) { attn_bwd_pre_body<true>(a); }

// Grid: (key tile, kv head) pairs. For key tiles split over several units, sums the units' fp32
// partials in chunk order (deterministic) and writes bf16 dK (times the softmax scale) and dV; other
// tiles were written directly by their unit.
template <bool F16>
__device__ __forceinline__ void attn_bwd_acc_body(AttnArgs a) {
  const int hkv = blockIdx.x % a.hkv;
  const int64_t n = blockIdx.x / a.hkv;
  const int chunks = a.plan.b_chunks[n];
  if (chunks <= 1) return;
  const int64_t slot = a.nk * a.hkv * kHeadDim;
  // Every slot of an element is requested before the first add (the slot count is at most
  // kMaxChunks), and four elements per thread are in flight at once; the sum still runs over the
  // slots in unit order.
#pragma unroll 4
  for (int i = threadIdx.x; i < kBwdTileN * (kHeadDim / 4); i += blockDim.x) {
    const int64_t key = n * kBwdTileN + i / (kHeadDim / 4);
    const int d = (i % (kHeadDim / 4)) * 4;
    if (key >= a.nk) continue;
    const float* pk = a.ws_dk + (key * a.hkv + hkv) * kHeadDim + d;
    const float* pv = a.ws_dv + (key * a.hkv + hkv) * kHeadDim + d;
    f32x4 kc[kMaxChunks], vc[kMaxChunks];
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      if (c < chunks) {
        kc[c] = *reinterpret_cast<const f32x4*>(pk + c * slot);
        vc[c] = *reinterpret_cast<const f32x4*>(pv + c * slot);
      }
    }
    f32x4 k4 = kc[0], v4 = vc[0];
#pragma unroll
    for (int c = 1; c < kMaxChunks; ++c) {
      if (c < chunks) {
        k4 += kc[c];
        v4 += vc[c];
      }
    }
    u32x2 wk, wv;
    wk.x = pack_elem2<F16>(k4[0] * a.scale, k4[1] * a.scale);
    wk.y = pack_elem2<F16>(k4[2] * a.scale, k4[3] * a.scale);
    wv.x = pack_elem2<F16>(v4[0], v4[1]);
    wv.y = pack_elem2<F16>(v4[2], v4[3]);
    *reinterpret_cast<u32x2*>(a.dk + key * a.dkst + hkv * a.dksh + d) = wk;
    *reinterpret_cast<u32x2*>(a.dv + key * a.dvst + hkv * a.dvsh + d) = wv;
  }
}

__global__ void __launch_bounds__(256) attn_bwd_acc_kernel(AttnArgs a) { attn_bwd_acc_body<false>(a); }
__global__ void __launch_bounds__(256) attn_bwd_acc_f16_kernel(AttnArgs a) { attn_bwd_acc_body<true>(a); }

// ---------------------------------------------------------------------------------------------
// dQ: query-major, same traversal and K/V ring as the forward. dQ^T = K^T dS^T.
// ---------------------------------------------------------------------------------------------
template <bool F16>
__device__ __forceinline__ void dq_tile(const uint16_t* sk, const uint16_t* sv,
                                        const bf16x8 (&qf)[8], const bf16x8 (&df)[8],
                                        f32x16 (&dqacc)[4], float lse2, float delta, bool partial,
                                        const RowIntervals& iv, float scale_log2, int ro,
                                        const TrOffsets& tro, int g) {
  const float neg_lse2 = -lse2;
  // One 32-key half at a time: dS of the half goes straight into dQ (8 registers of dS live). A
  // half that no row of the tile sees (a draft tile's other block pair, keys across a document
  // boundary) is skipped: its P, and so its dS and its dQ terms, are exact zeros.
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if (partial && __ballot(iv.word(kb, g) != 0u) == 0ull) continue;
    bf16x8 dsb[2];
    f32x16 s, dp;
    mfma_chains2<kDqAhead, F16>(s, dp, RowOperand{sk + kb * 32 * kRowLd, ro},
                           RowOperand{sv + kb * 32 * kRowLd, ro}, qf, df);
    bf16x8 kcur[4];
    read_tr_first(kcur, sk + kb * 32 * kRowLd, tro);
    if (partial) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = masked_score(s[r], iv.word(kb, g), r);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(fmaf(s[r], scale_log2, neg_lse2));
      s[r] = p * (dp[r] - delta);
    }
    dsb[0] = pack_c_half<F16>(s, 0);
    dsb[1] = pack_c_half<F16>(s, 8);
    mfma_tr_blocks<2, F16>(dqacc, sk + kb * 32 * kRowLd, tro, kcur, dsb);
  }
}

template <int G, bool F16>
__device__ __forceinline__ void attn_bwd_dq_body(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) KvStageFwd ring[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wave >= 0 && wave < G);
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t m = a.plan.nmf - 1 - blockIdx.x / a.hkv;
  const int head = hkv * G + wave;
  const int64_t qrow = m * kTM + c;
  const bool valid_q = qrow < a.nq;
  const int64_t qsafe = valid_q ? qrow : a.nq - 1;

  const uint16_t* kbase = a.k + hkv * a.ksh;
  const uint16_t* vbase = a.v + hkv * a.vsh;
  const int nk = static_cast<int>(a.nk);
  ListWindow lw{a.plan.f_list + m * a.plan.nnf, a.plan.f_cnt[m], 0, 0};
  lw.load(0, lane);
  const KvTileLanes lanes(lane);
  auto issue = [&](uint32_t entry, int stage) __attribute__((always_inline)) {
    const int key0 = static_cast<int>(entry & ~kFullBit) * kTN;
    issue_kv_tile<G>(kbase, a.kst, vbase, a.vst, key0, nk, ring[stage], wave, lanes);
  };
  if (lw.count > 0) issue(lw.entry(0), 0);

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
  const int ro = row_operand_off(c, g);
  const TrOffsets tro(lane);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  lds_barrier();

  for (int t = 0; t < lw.count; ++t) {
    const uint32_t entry = lw.entry(t);
    if (t + 1 < lw.count) {
      if (t + 1 - lw.base == kWave) lw.load(t + 1, lane);  // nothing else in flight here
      issue(lw.entry(t + 1), (t + 1) & 1);
    }
    const KvStageFwd& st = ring[t & 1];
    int ro_t = ro;
    TrOffsets tro_t = tro;
    opaque(ro_t);
    opaque(tro_t.lo);
    opaque(tro_t.hi);
    RowIntervals iv;
    iv.at_tile(static_cast<int>((entry & ~kFullBit) * kTN), cb, ce, db, de);
    dq_tile<F16>(st.k, st.v, qf, df, dqacc, lse2, delta, !(entry & kFullBit), iv, a.scale_log2, ro_t,
            tro_t, g);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's loads of tile t+1 have landed
    lds_barrier();
  }
  if (valid_q) store_row_c<F16>(a.dq + qrow * a.dqst + head * a.dqsh, dqacc, a.scale, g);
}

template <int G>
__global__ void __launch_bounds__(kWave * G, 2) attn_bwd_dq_kernel(AttnArgs a) { attn_bwd_dq_body<G, false>(a); }
template <int G>
__global__ void __launch_bounds__(kWave * G, 2) attn_bwd_dq_f16_kernel(AttnArgs a) { attn_bwd_dq_body<G, true>(a); }

// ---------------------------------------------------------------------------------------------
// dK / dV: key-major. A workgroup owns one 128-key tile and walks one chunk of the (descending)
// list of query tiles that see it; inside each query tile it visits all G heads of the KV group,
// so dK/dV are reduced over the GQA group in registers. A key tile covered by one unit is written
// directly; one split over several units writes each unit's fp32 partial to its own slot, and the
// finalize sums the slots in unit order.
//
// Eight waves in two roles share each 32-key slice w = wave % 4:
//   P waves (0-3):  S = Q K^T (K slice in registers), P = exp2(S*scale*log2e - LSE2) masked,
//                   P -> LDS, dV += P^T dO;
//   dS waves (4-7): dP = dO V^T (V slice in registers), dS = P (dP - delta) with P from LDS,
//                   dK += dS^T Q.
// The two waves of a SIMD thus overlap one's softmax VALU work with the other's MFMAs. Each role
// finishes stage i-1 at the start of trip i from operands carried in registers over the barrier
// (the P wave's dV product; the dS wave's dS and dK), then starts stage i (S and P; dP), so that
// a trip begins with MFMAs instead of every wave waiting on the same burst of LDS reads, and the
// two waves of a SIMD start with complementary work (MFMAs / VALU). Q/dO rows and the row scalars
// cycle through four LDS stages, straight from global memory into LDS (global_load_lds_dwordx4:
// no staging registers): stage i is read during trip i only; the dS waves load Q rows and row
// scalars into stage i+2 at the start of trip i, the P waves load dO rows into stage i+3 at the
// end of theirs. One barrier per trip.
// ---------------------------------------------------------------------------------------------
template <bool P>
struct Role {
  static constexpr bool value = P;
};

constexpr int kDkdvWaves = 2 * kKvWaves;
constexpr int kDkdvStages = 4;

struct KvStage {
  uint16_t q[kBwdTileM * kRowLd];     // swizzled rows
  uint16_t dout[kBwdTileM * kRowLd];
  float lse2[kBwdTileM];               // lse2 and delta are filled by one 64-lane load
  float delta[kBwdTileM];
  int32_t ends[4][kBwdTileM];          // cb, ce, db, de of each row (two 64-lane loads)
  uint32_t mask[kKvWaves][kBwdTileM];  // bit c of [w][row]: key 32w + c of the tile is visible
};
static_assert(offsetof(KvStage, delta) == offsetof(KvStage, lse2) + 4 * kBwdTileM, "layout");
static_assert(offsetof(KvStage, ends) == offsetof(KvStage, delta) + 4 * kBwdTileM, "layout");

// P of one iteration as the P wave's bf16 dV operand: [slice][C-register half][lane] (registers
// 8h .. 8h+7 of the lane, two per 32-bit word, low half first).
struct PExchange {
  uint4 p[kKvWaves][2][kWave];
};

// LDS read-ahead (k-steps) of the dK/dV kernel's S and dP chains.
constexpr int kDkdvAhead = 3;


// The first kDkdvAhead k-steps of an S / dP chain's A rows (LDS), read before other work.
template <typename Operand>
__device__ __forceinline__ void chain_first(uint4 (&x)[8], const Operand& ra) {
#pragma unroll
  for (int ds = 0; ds < kDkdvAhead; ++ds) x[ds] = ra.step(ds);
}

// acc = A x B over the 128-dim reduction: A rows from LDS (`x` holds the first kDkdvAhead k-steps,
// the rest are read kDkdvAhead steps ahead of their MFMA), B from registers.
template <bool F16 = false, typename Operand>
__device__ __forceinline__ f32x16 chain_rest(uint4 (&x)[8], const Operand& ra, const bf16x8 (&b)[8]) {
  f32x16 acc{};
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) {
    if (ds + kDkdvAhead < 8) x[ds + kDkdvAhead] = ra.step(ds + kDkdvAhead);
    acc = mfma32<F16>(as_bf16x8(x[ds]), b[ds], acc);
    ASPEC_STEP_FENCE();
  }
  return acc;
}

// The transposed fragments of a 32-row stage tile: rows (the reduction) 16*ks .. +15, columns
// 32*d .. +31.
__device__ __forceinline__ void read_tr_32(bf16x8 (&f)[2][4], const uint16_t* tile, const TrOffsets& tro) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int d = 0; d < 4; ++d) f[ks][d] = read_tr_operand(tile, tro, ks * 16, d * 32);
}

// acc[d] += F[ks][d] x B[ks] over a 32-row reduction, every operand in registers.
template <bool F16 = false>
__device__ __forceinline__ void mfma_regs_32(f32x16 (&acc)[4], const bf16x8 (&f)[2][4], const bf16x8 (&b)[2]) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int d = 0; d < 4; ++d) acc[d] = mfma32<F16>(f[ks][d], b[ks], acc[d]);
}

// What each role carries over the barrier from one trip to the next: the operands of the products
// that finish its previous stage, so that a trip starts with MFMAs from registers instead of
// waiting on LDS reads that every wave of the workgroup issues at the same moment.
struct PCarry {   // P wave: P of its previous stage (dV's B operand) and that stage's dO^T fragments
  bf16x8 p[2];
  bf16x8 d[2][4];
};
struct DsCarry {  // dS wave: dP of its previous stage, that stage's Q^T fragments and delta
  f32x16 dp;
  bf16x8 q[2][4];
  f32x4 delta[4];
};

// P wave, one trip: dV += P^T dO of the previous stage (carried operands), then, on a live stage:
// S = Q K^T (K slice in registers), the stage's dO^T fragments (read under the softmax), and
// P = exp2(S*scale*log2e - LSE2) masked, to LDS for the dS wave and into the carry. Rows at or
// past `valid` hold copies of a real row and get an empty mask. `key_base` is the slice's first
// key. A fully visible stage (a full tile with all rows real) skips the visibility words and the
// mask.
template <bool F16>
__device__ __forceinline__ void dkdv_p_step(KvStage& s, PExchange& px, const bf16x8 (&kf)[8],
                                            f32x16 (&dvacc)[4], PCarry& cy, bool live,
                                            float scale_log2, int w, int valid, bool all_visible,
                                            int key_base, const RowOffsets& ro,
                                            const TrOffsets& tro, int lane) {
  const int g = lane >> 5;
  const int c = lane & 31;
  uint4 x[8];
  f32x4 l4[4];
  if (live) {
    chain_first(x, RowOperandR{s.q, ro});
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) l4[rq] = *reinterpret_cast<const f32x4*>(s.lse2 + rq * 8 + g * 4);
  }
  ASPEC_STEP_FENCE();
  mfma_regs_32<F16>(dvacc, cy.d, cy.p);
  ASPEC_STEP_FENCE();
  if (!live) return;
  if (!all_visible) {
    if (lane < kBwdTileM) {  // visibility word of row `lane` for this slice
      const uint32_t bits = interval_bits(s.ends[0][lane], s.ends[1][lane], key_base) |
                            interval_bits(s.ends[2][lane], s.ends[3][lane], key_base);
      s.mask[w][lane] = lane < valid ? bits : 0u;
    }
    __builtin_amdgcn_wave_barrier();
  }
  f32x16 sacc = chain_rest<F16>(x, RowOperandR{s.q, ro}, kf);  // rows: queries, lane: key
  read_tr_32(cy.d, s.dout, tro);
  ASPEC_STEP_FENCE();
  if (all_visible) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq)
#pragma unroll
      for (int j = 0; j < 4; ++j) sacc[rq * 4 + j] = fast_exp2(sacc[rq * 4 + j] * scale_log2 - l4[rq][j]);
  } else {
    u32x4 m4[4];
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) m4[rq] = *reinterpret_cast<const u32x4*>(&s.mask[w][rq * 8 + g * 4]);
#pragma unroll
    for (int rq = 0; rq < 4; ++rq)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p = fast_exp2(sacc[rq * 4 + j] * scale_log2 - l4[rq][j]);
        const int keep = __builtin_amdgcn_sbfe(static_cast<int>(m4[rq][j]), c, 1);  // 0 or -1
        sacc[rq * 4 + j] = __int_as_float(__float_as_int(p) & keep);
      }
  }
  cy.p[0] = pack_c_half<F16>(sacc, 0);
  cy.p[1] = pack_c_half<F16>(sacc, 8);
  px.p[w][0][lane] = __builtin_bit_cast(uint4, cy.p[0]);
  px.p[w][1][lane] = __builtin_bit_cast(uint4, cy.p[1]);
}

// dS wave, one trip: dS = P (dP - delta) and dK += dS^T Q for the stage of its previous trip (dP,
// delta and the Q^T fragments carried, P from the P wave's exchange buffer: the bf16 P the dV
// product used; dS is rounded to bf16 for the dK product in any case); then, on a live stage:
// dP = dO V^T (V slice in registers) and the stage's Q^T fragments and delta.
template <bool F16>
__device__ __forceinline__ void dkdv_ds_step(const KvStage& s, const PExchange& px,
                                             const bf16x8 (&vf)[8], f32x16 (&dkacc)[4],
                                             DsCarry& cy, bool live, int w, const RowOffsets& ro,
                                             const TrOffsets& tro, int lane) {
  const int g = lane >> 5;
  const uint4 ph[2] = {px.p[w][0][lane], px.p[w][1][lane]};
  uint4 x[8];
  if (live) chain_first(x, RowOperandR{s.dout, ro});
  ASPEC_STEP_FENCE();
  f32x16 dp = cy.dp;
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
    const uint4& h = ph[rq >> 1];
    const uint32_t lo = (rq & 1) ? h.z : h.x;
    const uint32_t hi = (rq & 1) ? h.w : h.y;
    f32x4 p4;
    if constexpr (F16) {
      p4 = f32x4{elem_to_f32<true>(static_cast<uint16_t>(lo)), elem_to_f32<true>(static_cast<uint16_t>(lo >> 16)),
                 elem_to_f32<true>(static_cast<uint16_t>(hi)), elem_to_f32<true>(static_cast<uint16_t>(hi >> 16))};
    } else {
      p4 = f32x4{__uint_as_float(lo << 16), __uint_as_float(lo & 0xffff0000u),
                 __uint_as_float(hi << 16), __uint_as_float(hi & 0xffff0000u)};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) dp[rq * 4 + j] = p4[j] * (dp[rq * 4 + j] - cy.delta[rq][j]);
  }
  const bf16x8 dd[2] = {pack_c_half<F16>(dp, 0), pack_c_half<F16>(dp, 8)};
  mfma_regs_32<F16>(dkacc, cy.q, dd);
  ASPEC_STEP_FENCE();
  if (!live) return;
  cy.dp = chain_rest<F16>(x, RowOperandR{s.dout, ro}, vf);
  read_tr_32(cy.q, s.q, tro);
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) cy.delta[rq] = *reinterpret_cast<const f32x4*>(s.delta + rq * 8 + g * 4);
}

// LDS of the dK/dV kernel: the stage ring and P exchange during the walk, then, for the epilogue,
// one 32-key x 128-dim fp32 tile per key slice.
struct DkdvShared {
  union {
    struct {
      KvStage st[kDkdvStages];
      PExchange px[2];
    } walk;
    float out[kKvWaves][kBwdTileM * kHeadDim];
  };
  int32_t list[kUnitListCap];  // the unit's query tiles (| kFullBit)
};

// Epilogue of one wave: its 32 keys x 128 dims (C layout: lane = key, registers = dims) pass
// through the LDS tile `t` (row = key; 16-byte chunk j of row k stored at chunk j ^ k, which keeps
// both the writes and the row reads bank-conflict free) so that every global write instruction
// covers one contiguous key row: a bf16 store of the whole row (direct) or an fp32 store of the
// unit's partial into its own slot (key tiles split over several units; no atomics).
template <bool F16>
__device__ __forceinline__ void dkdv_store(const f32x16 (&acc)[4], float* t, int64_t key_first,
                                           int64_t nk, bool direct, uint16_t* dst,
                                           int64_t dst_stride, float* ws, int64_t ws_stride,
                                           float mul, int lane) {
  const int g = lane >> 5;
  const int c = lane & 31;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int chunk = db * 8 + rq * 2 + g;  // dims db*32 + rq*8 + g*4 .. +3
      const f32x4 v = {acc[db][rq * 4 + 0], acc[db][rq * 4 + 1], acc[db][rq * 4 + 2],
                       acc[db][rq * 4 + 3]};
      *reinterpret_cast<f32x4*>(t + c * kHeadDim + ((chunk ^ c) << 2)) = v;
    }
  __builtin_amdgcn_wave_barrier();
  for (int k = 0; k < kBwdTileM; ++k) {
    const int64_t key = key_first + k;
    if (key >= nk) break;
    const float* row = t + k * kHeadDim;
    const f32x2_t v = *reinterpret_cast<const f32x2_t*>(row + (((lane >> 1) ^ k) << 2) + (lane & 1) * 2);
    if (direct)
      *reinterpret_cast<uint32_t*>(dst + key * dst_stride + 2 * lane) = pack_elem2<F16>(v[0] * mul, v[1] * mul);
    else
      *reinterpret_cast<f32x2_t*>(ws + key * ws_stride + 2 * lane) = v;
  }
}

template <int G, bool F16>
__device__ __forceinline__ void attn_bwd_dkdv_body(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) DkdvShared sh;
  KvStage& st0 = sh.walk.st[0];
  KvStage& st1 = sh.walk.st[1];
  KvStage& st2 = sh.walk.st[2];
  KvStage& st3 = sh.walk.st[3];
  PExchange& px0 = sh.walk.px[0];
  PExchange& px1 = sh.walk.px[1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool p_role = wave < kKvWaves;
  const int w = wave % kKvWaves;
  const int g = lane >> 5;
  const int c = lane & 31;
  const int hkv = blockIdx.x % a.hkv;
  const int64_t u = blockIdx.x / a.hkv;
  if (u >= a.plan.b_nunits[0]) return;
  const int32_t unit = __builtin_amdgcn_readfirstlane(a.plan.b_units[u]);
  const int64_t n = unit >> kUnitChunkBits;
  const int chunk = unit & ((1 << kUnitChunkBits) - 1);
  const int count = __builtin_amdgcn_readfirstlane(a.plan.b_cnt[n]);
  const int chunks = __builtin_amdgcn_readfirstlane(a.plan.b_chunks[n]);
  const int len = bwd_unit_len(count);
  const int first = chunk * len;
  const int ntiles = max(0, min(count, first + len) - first);
  const int iters = ntiles * G;
  const int32_t* list = a.plan.b_list + n * a.plan.nmb;
  const int64_t key0 = n * kBwdTileN;
  // The unit's query tiles (| kFullBit) are staged in LDS, then held 128 at a time in two window
  // registers (lane j: entry wbase + j and wbase + 64 + j) and read with readlane in the loop: no
  // memory access there besides the stage loads.
  for (int j = tid; j < ntiles; j += kWave * kDkdvWaves) sh.list[j] = list[first + j];
  __syncthreads();
  int wbase = 0;
  int win0 = lane < ntiles ? sh.list[lane] : 0;
  int win1 = 64 + lane < ntiles ? sh.list[64 + lane] : 0;
  auto tile_entry = [&](int t) __attribute__((always_inline)) -> uint32_t {  // wbase <= t < wbase + 128
    const int r = t - wbase;
    const int e0 = __builtin_amdgcn_readlane(win0, r & 63);
    const int e1 = __builtin_amdgcn_readlane(win1, r & 63);
    return static_cast<uint32_t>(r < 64 ? e0 : e1);
  };
  auto advance_window = [&](int t) __attribute__((always_inline)) {  // makes t < wbase + 64
    if (t - wbase >= 64) {
      wbase += 64;
      win0 = win1;
      win1 = wbase + 64 + lane < ntiles ? sh.list[wbase + 64 + lane] : 0;
    }
  };

  // This wave's B operand for the whole walk: K (P waves) or V (dS waves) rows of its 32 keys.
  const int64_t key = key0 + w * 32 + c;
  const bool valid_k = key < a.nk;
  const int64_t ksafe = valid_k ? key : a.nk - 1;
  bf16x8 kvf[8];
  load_row_frag(kvf, p_role ? a.k + ksafe * a.kst + hkv * a.ksh : a.v + ksafe * a.vst + hkv * a.vsh,
                valid_k, g);
  f32x16 acc[4] = {};
  const RowOffsets ro(lane);
  const TrOffsets tro(lane);

  // The sources of this wave's stage loads are fixed for the whole walk: computed once and held in
  // SGPRs, behind an empty asm so that the compiler cannot re-derive them from the kernel arguments
  // inside the walk (each such reload is a scalar load whose wait also drains the wave's
  // outstanding LDS reads). P waves load dO rows, dS waves Q rows and the row scalars.
  const int64_t nq = opaque_s(a.nq);
  const float scale_log2 = opaque_s(a.scale_log2);
  const uint16_t* const rows_h0 = opaque_s(p_role ? a.dout + static_cast<int64_t>(hkv) * G * a.dosh
                                                  : a.q + static_cast<int64_t>(hkv) * G * a.qsh);
  const int64_t rows_tok = opaque_s(p_role ? a.dost : a.qst);
  const int64_t rows_head = opaque_s(p_role ? a.dosh : a.qsh);
  const uint32_t rows_tok2 = static_cast<uint32_t>(rows_tok * 2);
  const float* const delta_h0 = opaque_s(a.ws_delta + static_cast<int64_t>(hkv) * G * a.nq);
  const int32_t* const ends_w = a.ends + static_cast<int64_t>(max(w * 2 - 1, 0)) * nq;
  // Byte distance of the lanes 32-63 array: lse2 follows delta ([Hq][Nq] each), endpoint row e+1
  // follows row e.
  const uint32_t lane_half_ws = lane < 32 ? static_cast<uint32_t>(a.ws_lse2 - a.ws_delta) * 4u : 0u;
  const uint32_t lane_half_ends = lane < 32 ? 0u : static_cast<uint32_t>(a.nq) * 4u;
  auto row_base = [&](int it, int64_t& q0, int& h, int& valid) __attribute__((always_inline)) {
    q0 = static_cast<int64_t>(tile_entry(it / G) & ~kFullBit) * kBwdTileM;
    h = it % G;
    valid = static_cast<int>(min<int64_t>(kBwdTileM, nq - q0));
  };
  // Loads of iteration `it` into a stage, split by role so that no wave queues behind the whole
  // stage in the CU's address unit: dS wave w moves Q rows 8w .. 8w+7 (and dS waves 0-2 the row
  // scalars) at the start of a trip, into the stage two ahead; P wave w moves dO rows 8w .. 8w+7
  // at the end of its trip, after its softmax, into the stage three ahead (the one read during the
  // previous trip, free once that trip's barrier has passed), when the dS waves' loads have left
  // the address unit. Lane l lands at physical chunk l % 16 of its row, so it fetches the logical
  // chunk swizzled there; rows past the tensor repeat its last row.
  const int lrow_a = w * 8 + (lane >> 4), lrow_b = lrow_a + 4;
  const uint32_t lcol_a2 = static_cast<uint32_t>(((lane & 15) ^ swz(lrow_a)) * 8) * 2u;
  const uint32_t lcol_b2 = static_cast<uint32_t>(((lane & 15) ^ swz(lrow_b)) * 8) * 2u;
  const bool three_loads = !p_role && w < 3;  // two row loads + one scalar load
  auto issue = [&](int it, KvStage& sb) __attribute__((always_inline)) {
    int64_t q0;
    int h, valid;
    row_base(it, q0, h, valid);
    const uint32_t ra = static_cast<uint32_t>(min(lrow_a, valid - 1));
    const uint32_t rb = static_cast<uint32_t>(min(lrow_b, valid - 1));
    const uint16_t* rb_base = rows_h0 + q0 * rows_tok + h * rows_head;
    uint16_t* dst = (p_role ? sb.dout : sb.q) + w * 8 * kRowLd;
    lds_load16_at(rb_base, ra * rows_tok2 + lcol_a2, dst);
    lds_load16_at(rb_base, rb * rows_tok2 + lcol_b2, dst + 4 * kRowLd);
    if (p_role) return;
    const uint32_t r4 = static_cast<uint32_t>(min(lane & 31, valid - 1)) * 4u;
    if (w == 0) {
      lds_load4_at(delta_h0 + h * nq + q0, r4 + lane_half_ws, sb.lse2);
    } else if (w < 3) {
      lds_load4_at(ends_w + q0, r4 + lane_half_ends, sb.ends[(w - 1) * 2]);
    }
  };
  // Before the barrier that ends trip i, this wave's loads of stage i+1 have landed; `later`
  // counts its stages after i+1 already issued (dS waves: i+2; P waves: i+2 and i+3).
  auto wait_loads = [&](int later) __attribute__((always_inline)) {
    if (p_role) {
      if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
      else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));
      else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    } else {
      if (later == 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      else if (three_loads) __builtin_amdgcn_s_waitcnt(vmcnt_imm(3));
      else __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));
    }
  };
  // The edge trips (dS waves at trip 0, P waves at trip iters) finish a stage of zeros: the carries
  // start zeroed and P buffer 1 is zero-filled. Their contributions are exact zeros, and no
  // accumulator is merged across a branch inside the walk.
  {
    constexpr int np = static_cast<int>(sizeof(PExchange) / 16);
    static_assert(sizeof(PExchange) % 16 == 0, "16-byte fills");
    uint4* zp = reinterpret_cast<uint4*>(&px1);
    for (int i = tid; i < np; i += kWave * kDkdvWaves) zp[i] = make_uint4(0, 0, 0, 0);
  }
  if (iters > 0) issue(0, st0);
  if (iters > 1) issue(1, st1);
  if (p_role && iters > 2) issue(2, st2);
  wait_loads(p_role ? (iters > 1) + (iters > 2) : (iters > 1));  // stage 0 has landed
  lds_barrier();

  // Trip i (stage ring position i % 4): P waves finish stage i-1 (dV) and compute P of stage i;
  // dS waves finish stage i-1 (dS, dK) and compute dP of stage i; loads of iteration i+2 go into
  // stage i+2. Stage i is read only during trip i. Each role runs its own copy of the walk (same
  // trips, same barriers).
  PCarry pc{};
  DsCarry dc{};
  auto trip = [&](auto role, int i, KvStage& s_cur, KvStage& s_ld, KvStage& s_nx,
                  PExchange& x_cur, PExchange& x_prv) __attribute__((always_inline)) {
    advance_window(i / G);
    if (!p_role && i + 2 < iters) issue(i + 2, s_ld);
    TrOffsets tro_t = tro;
    opaque(tro_t.lo);
    opaque(tro_t.hi);
    const bool live = i < iters;
    if constexpr (decltype(role)::value) {
      int64_t q0;
      int h, valid;
      row_base(i, q0, h, valid);
      const bool full = (tile_entry(i / G) & kFullBit) != 0;
      dkdv_p_step<F16>(s_cur, x_cur, kvf, acc, pc, live, scale_log2, w, valid,
                  full && valid == kBwdTileM, static_cast<int>(key0) + w * 32, ro, tro_t, lane);
    } else {
      dkdv_ds_step<F16>(s_cur, x_prv, kvf, acc, dc, live, w, ro, tro_t, lane);
    }
    if (p_role && i + 3 < iters) issue(i + 3, s_nx);
    wait_loads(p_role ? (i + 2 < iters) + (i + 3 < iters) : (i + 2 < iters));
    lds_barrier();
  };
  // The break tests read the trip count through an empty asm: when G divides the unroll factor the
  // optimizer would otherwise drop three of them and merge three trips into one block, whose
  // register allocation spills.
  int stop = iters;
  asm volatile("" : "+s"(stop));
  auto walk = [&](auto role) __attribute__((always_inline)) {
    for (int i = 0; i <= iters; i += 4) {
      trip(role, i, st0, st2, st3, px0, px1);
      if (i + 1 > stop) break;
      trip(role, i + 1, st1, st3, st0, px1, px0);
      if (i + 2 > stop) break;
      trip(role, i + 2, st2, st0, st1, px0, px1);
      if (i + 3 > stop) break;
      trip(role, i + 3, st3, st1, st2, px1, px0);
    }
  };
  if (p_role)
    walk(Role<true>{});
  else
    walk(Role<false>{});
  // Epilogue in the walk's LDS (every load has landed): P waves (dV) first, then dS waves (dK).
  const bool direct = chunks == 1;
  const int64_t ws_stride = static_cast<int64_t>(a.hkv) * kHeadDim;
  const int64_t ws_slot = static_cast<int64_t>(chunk) * a.nk * ws_stride + hkv * kHeadDim;
  const int64_t key_first = key0 + w * 32;
  if (p_role)
    dkdv_store<F16>(acc, sh.out[w], key_first, a.nk, direct, a.dv + hkv * a.dvsh, a.dvst,
               a.ws_dv + ws_slot, ws_stride, 1.f, lane);
  lds_barrier();
  if (!p_role)
    dkdv_store<F16>(acc, sh.out[w], key_first, a.nk, direct, a.dk + hkv * a.dksh, a.dkst,
               a.ws_dk + ws_slot, ws_stride, a.scale, lane);
}

template <int G>
__global__ void __launch_bounds__(kWave * kDkdvWaves) attn_bwd_dkdv_kernel(AttnArgs a) { attn_bwd_dkdv_body<G, false>(a); }
template <int G>
__global__ void __launch_bounds__(kWave * kDkdvWaves) attn_bwd_dkdv_f16_kernel(AttnArgs a) { attn_bwd_dkdv_body<G, true>(a); }

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
  if ((a.kst > 0 && a.kst >= (1LL << 30) / kBwdTileN) || (a.vst > 0 && a.vst >= (1LL << 30) / kBwdTileN))
    return set_error(ASPEC_ERR_UNSUPPORTED, "K/V token stride too large for 32-bit tile offsets");
  if ((a.qst > 0 && a.qst >= (1LL << 30) / kBwdTileM) || (a.dost > 0 && a.dost >= (1LL << 30) / kBwdTileM))
    return set_error(ASPEC_ERR_UNSUPPORTED, "Q/dO token stride too large for 32-bit tile offsets");
  if (a.nk >= (1LL << 31) - kBwdTileN)
    return set_error(ASPEC_ERR_INVALID, "too many keys for int32 tile indexing");
  if (a.nq * a.hq >= (1LL << 29))
    return set_error(ASPEC_ERR_UNSUPPORTED, "too many query rows x heads for 32-bit workspace offsets");
  return ASPEC_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool stride_ok(int64_t s) { return s % 8 == 0; }

// Element type of the attention entry points (the ASPEC_MASK_* codes of include/aspec_amd.h).
constexpr int kDtypeBf16 = 4;
constexpr int kDtypeF16 = 5;

int check_dtype(int dtype) {
  if (dtype != kDtypeBf16 && dtype != kDtypeF16)
    return set_error(ASPEC_ERR_UNSUPPORTED, "DSpark attention computes in bf16 or fp16 (dtype code %d)", dtype);
  return ASPEC_OK;
}

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
                                     int dtype, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
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
  if (dtype == kDtypeF16) {
    ASPEC_GROUP_DISPATCH(attn_fwd_f16_kernel, a.group, grid, s, a);
  } else {
    ASPEC_GROUP_DISPATCH(attn_fwd_kernel, a.group, grid, s, a);
  }
  return check_launch("attn_fwd_kernel");
}

extern "C" int aspec_dspark_attn_bwd_workspace_bytes(int64_t num_queries, int64_t num_keys,
                                                     int64_t q_heads, int64_t kv_heads,
                                                     size_t* bytes) {
  if (num_queries <= 0 || num_keys <= 0 || q_heads <= 0 || kv_heads <= 0 || !bytes)
    return set_error(ASPEC_ERR_INVALID, "workspace size needs positive sizes");
  *bytes = static_cast<size_t>(2 * num_queries * q_heads +
                               2 * static_cast<int64_t>(kMaxChunks) * num_keys * kv_heads * kHeadDim) *
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
    void* workspace, int dtype, void* stream) {
  if (stages <= 0 || stages > 15) return set_error(ASPEC_ERR_INVALID, "backward stage mask must be 1..15");
  if (int rc = check_dtype(dtype)) return rc;
  const bool f16 = dtype == kDtypeF16;
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
  a.ws_dv = a.ws_dk + static_cast<int64_t>(kMaxChunks) * num_keys * kv_heads * kHeadDim;
  a.plan = plan_view(const_cast<void*>(plan), num_queries, num_keys);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 acc_grid(static_cast<uint32_t>(a.plan.nnb * a.hkv));

  if (stages & 1) {
    const int64_t pre_threads = num_queries * q_heads * 16;
    const dim3 grid(static_cast<uint32_t>((pre_threads + 255) / 256));
    if (f16)
      hipLaunchKernelGGL(attn_bwd_pre_f16_kernel, grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(attn_bwd_pre_kernel, grid, dim3(256), 0, s, a);
    if ((rc = check_launch("attn_bwd_pre_kernel"))) return rc;
  }
  if (stages & 2) {
    const dim3 grid(static_cast<uint32_t>(a.plan.nmf * a.hkv));
    if (f16) {
      ASPEC_GROUP_DISPATCH(attn_bwd_dq_f16_kernel, a.group, grid, s, a);
    } else {
      ASPEC_GROUP_DISPATCH(attn_bwd_dq_kernel, a.group, grid, s, a);
    }
    if ((rc = check_launch("attn_bwd_dq_kernel"))) return rc;
  }
  if (stages & 4) {
    const dim3 grid(static_cast<uint32_t>(a.plan.max_units * a.hkv)), block(kWave * kDkdvWaves);
    // the group size is a compile-time constant inside the walk
#define ASPEC_DKDV_DISPATCH(KERNEL)                                                   \
  switch (a.group) {                                                                 \
    case 1: hipLaunchKernelGGL(KERNEL<1>, grid, block, 0, s, a); break;              \
    case 2: hipLaunchKernelGGL(KERNEL<2>, grid, block, 0, s, a); break;              \
    case 3: hipLaunchKernelGGL(KERNEL<3>, grid, block, 0, s, a); break;              \
    case 4: hipLaunchKernelGGL(KERNEL<4>, grid, block, 0, s, a); break;              \
    case 5: hipLaunchKernelGGL(KERNEL<5>, grid, block, 0, s, a); break;              \
    case 6: hipLaunchKernelGGL(KERNEL<6>, grid, block, 0, s, a); break;              \
    case 7: hipLaunchKernelGGL(KERNEL<7>, grid, block, 0, s, a); break;              \
    default: hipLaunchKernelGGL(KERNEL<8>, grid, block, 0, s, a); break;             \
  }
    if (f16) {
      ASPEC_DKDV_DISPATCH(attn_bwd_dkdv_f16_kernel)
    } else {
      ASPEC_DKDV_DISPATCH(attn_bwd_dkdv_kernel)
    }
#undef ASPEC_DKDV_DISPATCH
    if ((rc = check_launch("attn_bwd_dkdv_kernel"))) return rc;
  }
  if (stages & 8) {
    if (f16)
      hipLaunchKernelGGL(attn_bwd_acc_f16_kernel, acc_grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(attn_bwd_acc_kernel, acc_grid, dim3(256), 0, s, a);
    rc = check_launch("attn_bwd_acc_kernel");
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
    void* workspace, int dtype, void* stream) {
  return aspec_dspark_attn_bwd_stages(
      15, q, q_stride_token, q_stride_head, k, k_stride_token, k_stride_head, v, v_stride_token,
      v_stride_head, out, o_stride_token, o_stride_head, dout, do_stride_token, do_stride_head,
      lse, dlse, endpoints, plan, num_queries, num_keys, q_heads, kv_heads, head_dim, scale, dq,
      dq_stride_token, dq_stride_head, dk, dk_stride_token, dk_stride_head, dv, dv_stride_token,
      dv_stride_head, workspace, dtype, stream);
}
