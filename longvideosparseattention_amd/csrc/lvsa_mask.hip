// Frame-mask builder, block plan and frame gather for the LVSA hot path (gfx950).
//
//   lvsa_mask_build   one work-group derives the anchor/keyframe/window pattern
//                     and writes the frame-level CSR (bit-exact with the
//                     reference FlashInfer CSR), per-frame window bounds and
//                     the frame relation as bitmaps.
//   lvsa_plan_build   refines a frame relation to canonical token blocks:
//                     per query tile, the active key blocks (CSR) and a mask
//                     descriptor per block.  count -> scan -> fill, all on the
//                     stream, no host synchronisation.
//   lvsa_gather_frames packs whole frames of K/V rows (build_global_kv).
//
// All three are integer / byte work, bounded by latency (mask, plan) or HBM
// bandwidth (gather); none of them touches MFMA.
#include "lvsa_common.h"

#include <cstring>
#include <mutex>
#include <string>

namespace lvsa {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

namespace {

constexpr int kMaskThreads = 1024;
constexpr int kPlanThreads = 128;
constexpr int kScanThreads = 1024;

// Exclusive scan of one int per thread across the work-group.
__device__ int block_exclusive_scan(int v, int* sh, int* total) {
  const int tid = threadIdx.x;
  sh[tid] = v;
  __syncthreads();
  for (int off = 1; off < (int)blockDim.x; off <<= 1) {
    int add = (tid >= off) ? sh[tid - off] : 0;
    __syncthreads();
    sh[tid] += add;
    __syncthreads();
  }
  const int incl = sh[tid];
  *total = sh[blockDim.x - 1];
  __syncthreads();
  return incl - v;
}

// Window bounds of query frame f (lvsa/sparse_attention.py:40-104).
// W = 0 gives the empty range (f, f-1); `expand` grows the adaptive window
// alternately left/right until it holds min(2W+1, T-|G|) non-global frames.
__device__ void frame_window(int f, int W, int T, bool expand, const uint8_t* gflag, int n_global,
                             int* lo_out, int* hi_out) {
  if (W == 0) {
    *lo_out = f;
    *hi_out = f - 1;
    return;
  }
  const int64_t w = W;
  int64_t lo = (int64_t)f - w < (int64_t)T - 1 - 2 * w ? (int64_t)f - w : (int64_t)T - 1 - 2 * w;
  if (lo < 0) lo = 0;
  int64_t hi = (int64_t)f + w > 2 * w ? (int64_t)f + w : 2 * w;
  if (hi > T - 1) hi = T - 1;
  if (expand) {
    const int64_t need = (2 * w + 1 < (int64_t)T - n_global) ? 2 * w + 1 : (int64_t)T - n_global;
    int64_t have = 0;
    for (int64_t x = lo; x <= hi; ++x) have += gflag[x] ? 0 : 1;
    bool left = true;
    int blocked = 0;
    while (have < need && blocked < 2) {
      int64_t added = -1;
      if (left && lo > 0) {
        added = --lo;
      } else if (!left && hi < T - 1) {
        added = ++hi;
      }
      left = !left;
      if (added < 0) {
        ++blocked;
        continue;
      }
      blocked = 0;
      if (!gflag[added]) ++have;
    }
  }
  *lo_out = (int)lo;
  *hi_out = (int)hi;
}

// compute_auto_kfi (lvsa/sparse_attention.py:132-195), evaluated by one
// work-group.  Budget B = max(n + 1, int(ref * scale)); T <= B gives 1.
// Otherwise the strict interval is the largest k in [1, T] whose grid
// {0, k, 2k, ...} < T together with the anchors 0..a-1 (a = min(n, T)) holds
// at least G = max(n, B - min(2W + 1, T)) frames, and that union has
// a + ceil(T/k) - ceil(a/k) frames, so each thread tests its share of k in
// O(1) each and the work-group takes the maximum.  The fallback is
// ceil(max(T - M, B - M) / max(B - M, 1)) with M = 2W + n, the result the
// larger of the two.  `budget` is int(ref * scale), truncated on the host.
struct KfiArgs {
  int T, window, n_first;
  int64_t budget;
};

__device__ int auto_kfi_block(const KfiArgs& k, int* s_best) {
  const int64_t T = k.T, n = k.n_first, W = k.window;
  const int64_t B = max(n + 1, k.budget);
  if (T <= B) return 1;                                   // uniform across the work-group
  const int64_t G = max(n, B - min(2 * W + 1, T));
  const int64_t a = max((int64_t)0, min(n, T));
  if (threadIdx.x == 0) *s_best = 1;
  __syncthreads();
  int best = 0;
  for (int64_t kk = threadIdx.x + 1; kk <= T; kk += blockDim.x) {
    const int64_t u = a + ceil_div(T, kk) - ceil_div(a, kk);
    if (u >= G) best = (int)kk;                           // ascending: the last hit is the largest
  }
  if (best) atomicMax(s_best, best);
  __syncthreads();
  const int strict = *s_best;
  const int64_t M = 2 * W + n;
  const int64_t num = max(T - M, B - M), den = max(B - M, (int64_t)1);
  const int64_t fallback = num >= 0 ? (num + den - 1) / den : num / den;   // ceil; C division truncates
  return (int)max((int64_t)strict, fallback);
}

__global__ __launch_bounds__(256) void auto_kfi_kernel(KfiArgs k, int32_t* out) {
  __shared__ int s_best;
  const int kfi = auto_kfi_block(k, &s_best);
  if (threadIdx.x == 0) *out = kfi;
}

struct MaskGeom {
  int64_t local, gts, budget;
  int T, P, first, n_local, n_rows, words;
};

// One 32-frame word of relation row `f`: bit set for global frames ("full"
// only) and for non-global window frames holding tokens on this rank (both).
__device__ inline void relation_word(const MaskGeom& g, int f, int lo, int hi, int w, const uint8_t* gflag,
                                     uint32_t* full, uint32_t* win) {
  uint32_t a = 0, b = 0;
  const int base = 32 * w;
  for (int bit = 0; bit < 32; ++bit) {
    const int fr = base + bit;
    if (fr >= g.T) break;
    if (gflag[fr]) {
      a |= 1u << bit;
    } else if (fr >= lo && fr <= hi) {
      const int64_t s = (int64_t)fr * g.P > g.gts ? (int64_t)fr * g.P : g.gts;
      const int64_t e = (int64_t)(fr + 1) * g.P < g.gts + g.local ? (int64_t)(fr + 1) * g.P : g.gts + g.local;
      if (s < e) {
        a |= 1u << bit;
        b |= 1u << bit;
      }
    }
  }
  *full = a;
  *win = b;
}

__global__ __launch_bounds__(kMaskThreads) void mask_build_kernel(lvsa_mask_params p, MaskGeom g,
                                                                  lvsa_mask_out out) {
  __shared__ uint8_t gflag[LVSA_MAX_FRAMES];
  __shared__ int16_t wlo[LVSA_MAX_FRAMES];
  __shared__ int16_t whi[LVSA_MAX_FRAMES];
  __shared__ int rowoff[LVSA_MAX_FRAMES + 2];
  __shared__ uint32_t uni[LVSA_BITMAP_WORDS];
  __shared__ int uprefix[LVSA_BITMAP_WORDS + 1];
  __shared__ int scan_sh[kMaskThreads];
  __shared__ int s_rowmax;
  __shared__ int s_kfi;

  const int T = g.T, tid = threadIdx.x, nt = blockDim.x;

  // 0. keyframe interval and offset: given, or derived here (device re-tune).
  int kfi = p.kfi, offset = p.offset;
  if (p.auto_kfi) {
    kfi = auto_kfi_block(KfiArgs{T, p.window, p.n_first, g.budget}, &s_kfi);
    offset = (int)(p.step % kfi);
  }

  // 1. global flags: anchors, boundary guards, rotated keyframe grid (mod T).
  for (int i = tid; i < T; i += nt)
    gflag[i] = (i < p.n_first) || ((p.guard_bits[i >> 5] >> (i & 31)) & 1u);
  for (int w = tid; w < LVSA_BITMAP_WORDS; w += nt) uni[w] = 0;
  if (tid == 0) s_rowmax = 0;
  __syncthreads();
  if (kfi > 0) {
    const int nkey = (T + kfi - 1) / kfi;
    for (int i = tid; i < nkey; i += nt) {
      int64_t x = ((int64_t)offset + (int64_t)i * kfi) % T;
      if (x < 0) x += T;
      gflag[x] = 1;
    }
  }
  __syncthreads();

  // 2. sorted global list via a scan over contiguous per-thread segments.
  const int seg = (T + nt - 1) / nt;
  const int s0 = min(T, tid * seg), s1 = min(T, s0 + seg);
  int cnt = 0;
  for (int i = s0; i < s1; ++i) cnt += gflag[i];
  int n_global;
  int pos = block_exclusive_scan(cnt, scan_sh, &n_global);
  for (int i = s0; i < s1; ++i)
    if (gflag[i]) out.global_frames[pos++] = i;
  for (int i = n_global + tid; i < T; i += nt) out.global_frames[i] = -1;

  // 3. window bounds of every frame.
  for (int f = tid; f < T; f += nt) {
    int lo, hi;
    frame_window(f, p.window, T, p.expand != 0, gflag, n_global, &lo, &hi);
    wlo[f] = (int16_t)lo;
    whi[f] = (int16_t)hi;
    out.window_bounds[2 * f] = lo;
    out.window_bounds[2 * f + 1] = hi;
  }
  __syncthreads();

  // 4. relation bitmaps of the local frames; union and row sizes of CSR rows.
  for (int r = tid; r < g.n_local; r += nt) {
    const int f = g.first + r;
    int nnz = 0;
    for (int w = 0; w < g.words; ++w) {
      uint32_t full, win;
      relation_word(g, f, wlo[f], whi[f], w, gflag, &full, &win);
      out.rel_full[(int64_t)r * g.words + w] = full;
      out.rel_window[(int64_t)r * g.words + w] = win;
      if (r < g.n_rows) {
        atomicOr(&uni[w], full);
        nnz += __popc(full);
      }
    }
    if (r < g.n_rows) {
      rowoff[r] = nnz;
      atomicMax(&s_rowmax, nnz);
    }
  }
  __syncthreads();

  // 5. compact ids = rank of a frame in the union of all CSR rows.
  if (tid == 0) {
    int acc = 0;
    for (int w = 0; w < g.words; ++w) {
      uprefix[w] = acc;
      acc += __popc(uni[w]);
    }
    uprefix[g.words] = acc;
  }
  __syncthreads();
  const int compact_n = uprefix[g.words];
  for (int w = tid; w < g.words; w += nt) {
    uint32_t u = uni[w];
    int k = uprefix[w];
    while (u) {
      const int b = __ffs(u) - 1;
      u &= u - 1;
      out.compact_frames[k++] = 32 * w + b;
    }
  }
  for (int i = compact_n + tid; i < T; i += nt) out.compact_frames[i] = -1;

  // 6. row pointers.
  const int rseg = (g.n_rows + nt - 1) / nt;
  const int r0 = min(g.n_rows, tid * rseg), r1 = min(g.n_rows, r0 + rseg);
  int rs = 0;
  for (int r = r0; r < r1; ++r) rs += rowoff[r];
  int nnz_total;
  int acc = block_exclusive_scan(rs, scan_sh, &nnz_total);
  for (int r = r0; r < r1; ++r) {
    const int c = rowoff[r];
    rowoff[r] = acc;
    out.frame_indptr[r] = acc;
    acc += c;
  }
  if (tid == 0) out.frame_indptr[g.n_rows] = nnz_total;
  __syncthreads();

  // 7. column ids, ascending per row.
  for (int r = tid; r < g.n_rows; r += nt) {
    const int f = g.first + r;
    int k = rowoff[r];
    for (int w = 0; w < g.words; ++w) {
      uint32_t full, win;
      relation_word(g, f, wlo[f], whi[f], w, gflag, &full, &win);
      const uint32_t uw = uni[w];
      while (full) {
        const int b = __ffs(full) - 1;
        full &= full - 1;
        out.frame_indices[k++] = uprefix[w] + __popc(uw & ((1u << b) - 1u));
      }
    }
  }
  if (tid == 0) {
    out.info[0] = nnz_total;
    out.info[1] = compact_n;
    out.info[2] = n_global;
    out.info[3] = g.n_rows;
    out.info[4] = g.n_local;
    out.info[5] = g.first;
    out.info[6] = s_rowmax;
    out.info[7] = kfi > 0 ? kfi : 0;
  }
}

// ───────────────────────────── block plan ──────────────────────────────────

struct PlanCtx {
  lvsa_plan_params p;
  int n_vt, n_tt, nkc, nxc;
};

__device__ inline uint32_t rel_word(const PlanCtx& c, int row, int w) {
  if (row < 0 || row >= c.p.rel_rows || w >= c.p.words) return 0u;
  return c.p.rel[(int64_t)row * c.p.words + w];
}

__device__ inline uint32_t rel_bit(const PlanCtx& c, int row, int64_t kf) {
  if (kf < 0) return 0u;
  return (rel_word(c, row, (int)(kf >> 5)) >> (kf & 31)) & 1u;
}

// Descriptor of a block of a dense source (text or extra rows): full, or a
// key tail.
__device__ inline uint32_t dense_desc(const PlanCtx& c, int64_t n, int64_t j) {
  const int64_t k0 = j * c.p.block_k;
  const int64_t kn = (n - k0) < c.p.block_k ? (n - k0) : c.p.block_k;
  if (kn == c.p.block_k) return make_desc(kKindNone, 0, 0, 0);
  return make_desc(kKindTwoPart, 0x5u, (uint32_t)kn, 255u);
}

// Descriptor of block j of the frame-structured source for the query tile
// holding rows [r0, r1) whose relation rows are qf0..qf1.
__device__ uint32_t frame_desc(const PlanCtx& c, int64_t r0, int qf0, int qf1, int64_t j) {
  const lvsa_plan_params& p = c.p;
  const int64_t k0 = j * p.block_k;
  const int64_t k1 = (k0 + p.block_k) < p.n_k ? (k0 + p.block_k) : p.n_k;
  const int64_t kfa = (p.k_tok0 + k0) / p.C, kfb = (p.k_tok0 + k1 - 1) / p.C;
  const bool tail = (k1 - k0) < p.block_k;
  const int nq = qf1 - qf0 + 1;
  const int64_t nk = kfb - kfa + 1 + (tail ? 1 : 0);
  if (nq <= 2 && nk <= 2) {
    const bool two = kfb > kfa;
    const int64_t kb = two ? (kfb * p.C - p.k_tok0 - k0) : (k1 - k0);
    const uint32_t alo = rel_bit(c, qf0, kfa), ahi = two ? rel_bit(c, qf0, kfb) : 0u;
    const uint32_t blo = rel_bit(c, qf1, kfa), bhi = two ? rel_bit(c, qf1, kfb) : 0u;
    // Row split inside the tile (1..block_q-1 <= 383: bits 16-24).  Without a
    // split both halves carry the same bits, so any value works; 255 is used.
    const int64_t qs = (nq == 2) ? ((int64_t)(qf1 + p.q_frame0) * p.R - p.q_tok0 - r0) : 255;
    const bool all = alo && blo && (kb >= p.block_k || (ahi && bhi));
    if (all) return make_desc(kKindNone, 0, 0, 0);
    return make_desc(kKindTwoPart, alo | (ahi << 1) | (blo << 2) | (bhi << 3), (uint32_t)kb, (uint32_t)qs);
  }
  if (!tail) {
    bool all = true;
    for (int q = qf0; q <= qf1 && all; ++q)
      for (int64_t kf = kfa; kf <= kfb && all; ++kf) all = rel_bit(c, q, kf) != 0u;
    if (all) return make_desc(kKindNone, 0, 0, 0);
  }
  return make_desc(kKindGeneric, 0, 0, 0);
}

template <bool kFill>
__global__ __launch_bounds__(kPlanThreads) void plan_tiles_kernel(PlanCtx c, int32_t* indptr, uint32_t* entries,
                                                                  int64_t cap) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= c.n_vt + c.n_tt) return;
  const lvsa_plan_params& p = c.p;
  int64_t pos = kFill ? (int64_t)indptr[t] : 0;
  const int64_t end = kFill ? (int64_t)indptr[t + 1] : 0;
  int64_t count = 0;
  auto emit = [&](uint32_t w0, uint32_t w1) {
    if (kFill && pos < end && pos < cap) {
      entries[2 * pos] = w0;
      entries[2 * pos + 1] = w1;
    }
    ++pos;
    ++count;
  };
  if (t < c.n_vt) {
    const int64_t r0 = (int64_t)t * p.block_q;
    const int64_t r1 = (r0 + p.block_q) < p.n_q ? (r0 + p.block_q) : p.n_q;
    const int qf0 = (int)((p.q_tok0 + r0) / p.R) - p.q_frame0;
    const int qf1 = (int)((p.q_tok0 + r1 - 1) / p.R) - p.q_frame0;
    int64_t jnext = 0;
    for (int w = 0; w < p.words; ++w) {
      uint32_t u = 0;
      for (int q = qf0; q <= qf1; ++q) u |= rel_word(c, q, w);
      while (u) {
        const int b = __ffs(u) - 1;
        u &= u - 1;
        const int64_t kf = 32 * (int64_t)w + b;
        int64_t a = kf * p.C - p.k_tok0, e = a + p.C;
        if (a < 0) a = 0;
        if (e > p.n_k) e = p.n_k;
        if (a >= e) continue;
        const int64_t jlo = a / p.block_k, jhi = (e - 1) / p.block_k;
        for (int64_t j = (jlo > jnext ? jlo : jnext); j <= jhi; ++j)
          emit((uint32_t)j, frame_desc(c, r0, qf0, qf1, j));
        if (jhi + 1 > jnext) jnext = jhi + 1;
      }
    }
  } else {
    for (int64_t j = 0; j < c.nkc; ++j) emit((uint32_t)j, dense_desc(c, p.n_k, j));
  }
  for (int64_t j = 0; j < c.nxc; ++j) emit(kSrcExtra | (uint32_t)j, dense_desc(c, p.n_x, j));
  if (!kFill) indptr[t + 1] = (int32_t)count;
}

// indptr[1..n] holds per-tile counts; turn it into row pointers, clamped to
// the entry capacity (status[0] = 1 when the bound was exceeded).
__global__ __launch_bounds__(kScanThreads) void plan_scan_kernel(int32_t* indptr, int n, int64_t cap,
                                                                 int32_t* status) {
  __shared__ int scan_sh[kScanThreads];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int seg = (n + nt - 1) / nt;
  const int a = min(n, tid * seg), b = min(n, a + seg);
  int s = 0;
  for (int i = a; i < b; ++i) s += indptr[i + 1];
  int total;
  int acc = block_exclusive_scan(s, scan_sh, &total);
  for (int i = a; i < b; ++i) {
    acc += indptr[i + 1];
    indptr[i + 1] = acc < cap ? acc : (int32_t)cap;
  }
  if (tid == 0) {
    indptr[0] = 0;
    status[0] = total > cap ? 1 : 0;
    status[1] = total;
  }
}

__global__ void plan_empty_kernel(int32_t* indptr, int32_t* status) {
  indptr[0] = 0;
  status[0] = 0;
  status[1] = 0;
}

// Rows of a block CSR -> relation bitmap (one thread per row).
__global__ __launch_bounds__(128) void csr_to_bitmap_kernel(const int32_t* indptr, const int32_t* indices,
                                                            int n_rows, int n_cols, int words, uint32_t* out,
                                                            int32_t* status) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n_rows) return;
  uint32_t* row = out + (int64_t)r * words;
  for (int w = 0; w < words; ++w) row[w] = 0u;
  const int a = indptr[r], b = indptr[r + 1];
  for (int e = a; e < b; ++e) {
    const int c = indices[e];
    if (c >= 0 && c < n_cols) {
      row[c >> 5] |= 1u << (c & 31);
    } else {
      status[0] = 1;  // column out of range: reported, not written
    }
  }
}

// ───────────────────────────── frame gather ────────────────────────────────

template <typename V>
__global__ __launch_bounds__(256) void gather_frames_kernel(const char* src, int64_t ss0, int64_t ss1,
                                                            int64_t ss2, char* dst, int64_t ds0, int64_t ds1,
                                                            int64_t ds2, const int32_t* frames, int P, int H,
                                                            int row_vecs) {
  const int64_t row = blockIdx.x;
  const int b = blockIdx.y;
  const int64_t i = row / P, t = row % P;
  const int64_t srow = (int64_t)frames[i] * P + t;
  const char* s = src + b * ss0 + srow * ss1;
  char* d = dst + b * ds0 + row * ds1;
  for (int x = threadIdx.x; x < H * row_vecs; x += blockDim.x) {
    const int h = x / row_vecs, v = x % row_vecs;
    reinterpret_cast<V*>(d + h * ds2)[v] = reinterpret_cast<const V*>(s + h * ss2)[v];
  }
}

}  // namespace
}  // namespace lvsa

using namespace lvsa;

extern "C" {

const char* lvsa_version(void) { return LVSA_AMD_VERSION; }

const char* lvsa_last_error(void) { return g_last_error.c_str(); }

// int(reference_frames * sparsity_scale) as Python computes it (a double
// product truncated toward zero); NaN is an error there too.
static int kfi_budget(int32_t reference_frames, double sparsity_scale, int64_t* budget) {
  const double prod = (double)reference_frames * sparsity_scale;
  LVSA_REQUIRE(prod == prod, LVSA_ERR_INVALID_ARG, "lvsa: sparsity_scale is NaN");
  *budget = prod >= 9.0e18 ? INT64_MAX : prod <= -9.0e18 ? INT64_MIN : (int64_t)prod;
  return LVSA_OK;
}

static int mask_geometry(const lvsa_mask_params* p, lvsa_mask_sizes* s, MaskGeom* g) {
  LVSA_REQUIRE(p != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_mask: null params");
  int rc = LVSA_OK;
  int64_t budget = 0;
  LVSA_REQUIRE(p->T >= 1 && p->T <= LVSA_MAX_FRAMES, LVSA_ERR_INVALID_ARG,
               "lvsa_mask: T=%d outside [1, %d]", p->T, LVSA_MAX_FRAMES);
  LVSA_REQUIRE(p->P >= 1, LVSA_ERR_INVALID_ARG, "lvsa_mask: P=%d must be >= 1", p->P);
  LVSA_REQUIRE(p->window >= 0, LVSA_ERR_INVALID_ARG, "lvsa_mask: window=%d must be >= 0", p->window);
  LVSA_REQUIRE(p->window <= 1 << 14, LVSA_ERR_INVALID_ARG, "lvsa_mask: window=%d too large", p->window);
  LVSA_REQUIRE(p->n_first >= 0, LVSA_ERR_INVALID_ARG, "lvsa_mask: n_first=%d must be >= 0", p->n_first);
  LVSA_REQUIRE(p->world >= 1 && p->rank >= 0 && p->rank < p->world, LVSA_ERR_INVALID_ARG,
               "lvsa_mask: rank=%d world=%d invalid", p->rank, p->world);
  const int64_t total = (int64_t)p->T * p->P;
  LVSA_REQUIRE(total % p->world == 0, LVSA_ERR_INVALID_ARG,
               "total_seq=%lld (T=%d x P=%d) must be divisible by world=%d.", (long long)total, p->T, p->P,
               p->world);
  if (p->auto_kfi) {
    LVSA_REQUIRE(p->step >= 0, LVSA_ERR_INVALID_ARG, "lvsa_mask: step=%lld must be >= 0", (long long)p->step);
    rc = kfi_budget(p->reference_frames, p->sparsity_scale, &budget);
    if (rc) return rc;
  }
  const int64_t local = total / p->world, gts = (int64_t)p->rank * local;
  const int first = (int)(gts / p->P), last = (int)((gts + local - 1) / p->P);
  s->local_seq = local;
  s->global_token_start = gts;
  s->n_rows = (int32_t)ceil_div(local, p->P);
  s->n_local = last - first + 1;
  s->words = (int32_t)ceil_div(p->T, 32);
  s->max_nnz = s->n_rows * p->T;
  if (g) {
    g->local = local;
    g->gts = gts;
    g->budget = budget;
    g->T = p->T;
    g->P = p->P;
    g->first = first;
    g->n_local = s->n_local;
    g->n_rows = s->n_rows;
    g->words = s->words;
  }
  return LVSA_OK;
}

int lvsa_mask_sizes_query(const lvsa_mask_params* p, lvsa_mask_sizes* out) {
  clear_error();
  LVSA_REQUIRE(out != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_mask_sizes_query: null output");
  return mask_geometry(p, out, nullptr);
}

int lvsa_mask_build(const lvsa_mask_params* p, const lvsa_mask_out* out, hipStream_t stream) {
  clear_error();
  lvsa_mask_sizes s;
  MaskGeom g;
  int rc = mask_geometry(p, &s, &g);
  if (rc) return rc;
  LVSA_REQUIRE(out != nullptr && out->frame_indptr && out->frame_indices && out->compact_frames &&
                   out->global_frames && out->window_bounds && out->rel_full && out->rel_window && out->info,
               LVSA_ERR_INVALID_ARG, "lvsa_mask_build: null output pointer");
  hipLaunchKernelGGL(mask_build_kernel, dim3(1), dim3(kMaskThreads), 0, stream, *p, g, *out);
  return launch_status("lvsa_mask_build");
}

int lvsa_auto_kfi(int32_t T, int32_t window, int32_t n_first, int32_t reference_frames, double sparsity_scale,
                  int32_t* kfi_out, hipStream_t stream) {
  clear_error();
  LVSA_REQUIRE(T >= 1, LVSA_ERR_INVALID_ARG, "lvsa_auto_kfi: T=%d must be >= 1", T);
  LVSA_REQUIRE(window >= 0 && window <= 1 << 28, LVSA_ERR_INVALID_ARG, "lvsa_auto_kfi: window=%d out of range",
               window);
  LVSA_REQUIRE(n_first >= 0, LVSA_ERR_INVALID_ARG, "lvsa_auto_kfi: n_first=%d must be >= 0", n_first);
  LVSA_REQUIRE(kfi_out != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_auto_kfi: null output");
  int64_t budget;
  const int rc = kfi_budget(reference_frames, sparsity_scale, &budget);
  if (rc) return rc;
  hipLaunchKernelGGL(auto_kfi_kernel, dim3(1), dim3(256), 0, stream, KfiArgs{T, window, n_first, budget}, kfi_out);
  return launch_status("lvsa_auto_kfi");
}

static int plan_ctx(const lvsa_plan_params* p, PlanCtx* c) {
  LVSA_REQUIRE(p != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_plan: null params");
  LVSA_REQUIRE(p->n_q >= 0 && p->n_k >= 0 && p->n_x >= 0 && p->n_tq >= 0, LVSA_ERR_INVALID_ARG,
               "lvsa_plan: negative length");
  LVSA_REQUIRE(p->block_q >= 1 && p->block_q <= 384 && p->block_k >= 1 && p->block_k <= 255,
               LVSA_ERR_INVALID_ARG, "lvsa_plan: block sizes (%d, %d) must lie in [1, 384] x [1, 255]",
               p->block_q, p->block_k);
  LVSA_REQUIRE(p->n_q == 0 || (p->R >= 1 && p->C >= 1 && p->rel != nullptr && p->words >= 1 && p->rel_rows >= 1),
               LVSA_ERR_INVALID_ARG, "lvsa_plan: video rows need a relation (R, C, rel, words, rel_rows)");
  LVSA_REQUIRE(p->q_tok0 >= 0 && p->k_tok0 >= 0, LVSA_ERR_INVALID_ARG, "lvsa_plan: negative token offset");
  if (p->n_q > 0) {
    // every query row needs a relation row: rows outside it would attend nothing
    const int64_t first = p->q_tok0 / p->R - p->q_frame0, last = (p->q_tok0 + p->n_q - 1) / p->R - p->q_frame0;
    LVSA_REQUIRE(first >= 0 && last < p->rel_rows, LVSA_ERR_INVALID_ARG,
                 "lvsa_plan: query rows map to relation rows [%lld, %lld], the relation has %d rows",
                 (long long)first, (long long)last, p->rel_rows);
  }
  c->p = *p;
  c->n_vt = (int)ceil_div(p->n_q, p->block_q);
  c->n_tt = (int)ceil_div(p->n_tq, p->block_q);
  c->nkc = (int)ceil_div(p->n_k, p->block_k);
  c->nxc = (int)ceil_div(p->n_x, p->block_k);
  return LVSA_OK;
}

int lvsa_plan_sizes_query(const lvsa_plan_params* p, int32_t max_row_frames, lvsa_plan_sizes* out) {
  clear_error();
  LVSA_REQUIRE(out != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_plan_sizes_query: null output");
  PlanCtx c;
  int rc = plan_ctx(p, &c);
  if (rc) return rc;
  int64_t per_video = 0;
  if (c.n_vt > 0) {
    const int64_t qframes = (p->block_q - 1) / p->R + 2;
    const int64_t rows = qframes < p->rel_rows ? qframes : p->rel_rows;
    const int64_t mr = max_row_frames > 0 ? max_row_frames : (int64_t)p->words * 32;
    const int64_t bound = rows * mr * (ceil_div(p->C, p->block_k) + 1);
    per_video = (bound < c.nkc ? bound : c.nkc) + c.nxc;
  }
  out->n_tiles = c.n_vt + c.n_tt;
  out->n_video_tiles = c.n_vt;
  out->max_entries = (int64_t)c.n_vt * per_video + (int64_t)c.n_tt * (c.nkc + c.nxc);
  out->workspace_bytes = 16;
  return LVSA_OK;
}

int lvsa_plan_build(const lvsa_plan_params* p, int32_t* tile_indptr, uint32_t* entries, int64_t max_entries,
                    void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  PlanCtx c;
  int rc = plan_ctx(p, &c);
  if (rc) return rc;
  LVSA_REQUIRE(tile_indptr && entries && workspace, LVSA_ERR_INVALID_ARG, "lvsa_plan_build: null pointer");
  LVSA_REQUIRE(workspace_bytes >= 16, LVSA_ERR_CAPACITY, "lvsa_plan_build: workspace of %lld bytes < 16",
               (long long)workspace_bytes);
  LVSA_REQUIRE(max_entries < (int64_t)INT32_MAX, LVSA_ERR_CAPACITY, "lvsa_plan_build: entry capacity too large");
  const int n = c.n_vt + c.n_tt;
  if (n == 0) {
    hipLaunchKernelGGL(plan_empty_kernel, dim3(1), dim3(1), 0, stream, tile_indptr, (int32_t*)workspace);
    return launch_status("lvsa_plan_build");
  }
  const dim3 grid((unsigned)ceil_div(n, kPlanThreads));
  hipLaunchKernelGGL(plan_tiles_kernel<false>, grid, dim3(kPlanThreads), 0, stream, c, tile_indptr, entries,
                     max_entries);
  hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, tile_indptr, n, max_entries,
                     (int32_t*)workspace);
  hipLaunchKernelGGL(plan_tiles_kernel<true>, grid, dim3(kPlanThreads), 0, stream, c, tile_indptr, entries,
                     max_entries);
  return launch_status("lvsa_plan_build");
}

int lvsa_csr_to_bitmap(const int32_t* indptr, const int32_t* indices, int32_t n_rows, int32_t n_cols,
                       uint32_t* bitmap, int32_t words, int32_t* status, hipStream_t stream) {
  clear_error();
  LVSA_REQUIRE(indptr && bitmap && status, LVSA_ERR_INVALID_ARG, "lvsa_csr_to_bitmap: null pointer");
  LVSA_REQUIRE(n_rows >= 0 && n_cols >= 0, LVSA_ERR_INVALID_ARG, "lvsa_csr_to_bitmap: negative size");
  LVSA_REQUIRE(words >= (n_cols + 31) / 32, LVSA_ERR_CAPACITY, "lvsa_csr_to_bitmap: %d words < %d columns", words,
               n_cols);
  hipLaunchKernelGGL(plan_empty_kernel, dim3(1), dim3(1), 0, stream, (int32_t*)status + 2, status);
  if (n_rows == 0) return launch_status("lvsa_csr_to_bitmap");
  LVSA_REQUIRE(indices != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_csr_to_bitmap: null indices");
  hipLaunchKernelGGL(csr_to_bitmap_kernel, dim3((unsigned)ceil_div(n_rows, 128)), dim3(128), 0, stream, indptr,
                     indices, n_rows, n_cols, words, bitmap, status);
  return launch_status("lvsa_csr_to_bitmap");
}

int lvsa_gather_frames(const void* src, const int64_t src_str[3], void* dst, const int64_t dst_str[3],
                       const int32_t* frames, int32_t n_frames, int32_t P, int32_t B, int32_t H, int32_t D,
                       int32_t elem_bytes, hipStream_t stream) {
  clear_error();
  LVSA_REQUIRE(src && dst && src_str && dst_str, LVSA_ERR_INVALID_ARG, "lvsa_gather_frames: null pointer");
  LVSA_REQUIRE(n_frames >= 0 && P >= 1 && B >= 1 && H >= 1 && D >= 1, LVSA_ERR_INVALID_ARG,
               "lvsa_gather_frames: bad sizes");
  LVSA_REQUIRE(elem_bytes == 2 || elem_bytes == 4, LVSA_ERR_UNSUPPORTED, "lvsa_gather_frames: elem_bytes=%d",
               elem_bytes);
  if (n_frames == 0) return LVSA_OK;
  LVSA_REQUIRE(frames != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_gather_frames: null frame list");
  const int64_t rows = (int64_t)n_frames * P;
  LVSA_REQUIRE(rows < (int64_t)INT32_MAX && B <= 65535, LVSA_ERR_INVALID_ARG, "lvsa_gather_frames: too large");
  const int64_t ss0 = src_str[0] * elem_bytes, ss1 = src_str[1] * elem_bytes, ss2 = src_str[2] * elem_bytes;
  const int64_t ds0 = dst_str[0] * elem_bytes, ds1 = dst_str[1] * elem_bytes, ds2 = dst_str[2] * elem_bytes;
  const int64_t row_bytes = (int64_t)D * elem_bytes;
  auto aligned = [&](int64_t a) { return (a % 16) == 0; };
  const bool v16 = aligned(row_bytes) && aligned(ss0) && aligned(ss1) && aligned(ss2) && aligned(ds0) &&
                   aligned(ds1) && aligned(ds2) && aligned((int64_t)(uintptr_t)src) &&
                   aligned((int64_t)(uintptr_t)dst);
  const dim3 grid((unsigned)rows, (unsigned)B);
  if (v16) {
    hipLaunchKernelGGL(gather_frames_kernel<int4>, grid, dim3(256), 0, stream, (const char*)src, ss0, ss1, ss2,
                       (char*)dst, ds0, ds1, ds2, frames, P, H, (int)(row_bytes / 16));
  } else if (elem_bytes == 4) {
    hipLaunchKernelGGL(gather_frames_kernel<int>, grid, dim3(256), 0, stream, (const char*)src, ss0, ss1, ss2,
                       (char*)dst, ds0, ds1, ds2, frames, P, H, (int)(row_bytes / 4));
  } else {
    hipLaunchKernelGGL(gather_frames_kernel<short>, grid, dim3(256), 0, stream, (const char*)src, ss0, ss1, ss2,
                       (char*)dst, ds0, ds1, ds2, frames, P, H, (int)(row_bytes / 2));
  }
  return launch_status("lvsa_gather_frames");
}

}  // extern "C"
