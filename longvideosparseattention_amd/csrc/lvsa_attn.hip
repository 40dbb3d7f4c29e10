// Block-sparse flash-attention forward for LVSA on gfx950 (MI355X): the C ABI
// entry point (lvsa_attn_fwd), its argument checks and the dispatch by head
// size.  The kernels are in lvsa_attn_kernels.h, instantiated per head size
// in lvsa_attn_d64.hip, lvsa_attn_d96.hip, lvsa_attn_d128.hip,
// lvsa_attn_d192.hip and lvsa_attn_d256.hip.
#include "lvsa_attn_kernels.h"

#include <cstdlib>
#include <cstring>
#include <mutex>

using namespace lvsa;

namespace {

// Key blocks (of 64 keys) per text chunk when a text tile is split: about a
// third of a Wan / HunyuanVideo video tile and below a CogVideoX one, so the
// chunks fill the launch's last round at a granularity finer than a tile
// (64 measured the same at CogVideoX and 0.3% slower at HunyuanVideo).
constexpr int kTextChunkBlocks = 128;
constexpr int kMaxTextChunks = 64;

// Text chunks per text tile for the arguments (1 = no split).
int text_chunks_of(const lvsa_attn_args* a) {
  if (a->n_tq == 0 || a->dtype == LVSA_FP32) return 1;   // the fp32 kernel runs text tiles whole
  const int64_t blocks = ceil_div(a->n_k, kBN) + ceil_div(a->n_x, kBN);
  const int64_t c = ceil_div(blocks, kTextChunkBlocks);
  return (int)(c < 1 ? 1 : (c > kMaxTextChunks ? kMaxTextChunks : c));
}

int64_t text_ws_bytes(const lvsa_attn_args* a, int chunks) {
  if (a->n_tq == 0 || chunks <= 1) return 0;
  return 4 * (text_ws_o_elems(chunks, a->B, a->H, a->n_tq, a->D) + 2LL * chunks * a->B * a->H * a->n_tq);
}

// Partials of the video split with `vsplit` slots per queue (O, then the
// (running max, row sum) pairs).
int64_t video_ws_bytes(const lvsa_attn_args* a, int vsplit) {
  if (vsplit <= 0) return 0;
  return 4 * (video_ws_o_elems(vsplit, a->block_q, a->D) + 2LL * kXcds * vsplit * 2 * a->block_q);
}

// Workspace of a call: the text-split partials (text_ws_bytes) at offset 0,
// the video-split partials (video_ws_bytes) after them at a 256-byte
// boundary, then the work-queue counters (kQueueBytes) at the next one.
int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }
int64_t video_offset(const lvsa_attn_args* a, int chunks) { return align256(text_ws_bytes(a, chunks)); }
int64_t queue_offset(const lvsa_attn_args* a, int chunks, int vsplit) {
  return align256(video_offset(a, chunks) + video_ws_bytes(a, vsplit));
}
int64_t ws_bytes(const lvsa_attn_args* a, int vsplit) {
  return queue_offset(a, text_chunks_of(a), vsplit) + kQueueBytes;
}

// Zero the work-queue counters (a kernel, not a memset, so the call can be
// captured in a HIP graph and replayed).
__global__ __launch_bounds__(64) void queue_reset_kernel(uint32_t* q) {
  if (threadIdx.x < 8) q[threadIdx.x * (kQueueStride / 4)] = 0u;
}

// Compute units of the current device (the persistent grid of the
// single-stream kernel), cached per device.
int cu_count() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cached[dev] = n;
  }
  return cached[dev];
}

// Whether a 16-bit head size 64 plan of 256-row tiles runs the dual map
// (LVSA_D64_WAVES=8 selects 8 waves of 32 rows instead, for comparisons).
bool dual_map(const lvsa_attn_args* a) {
  const char* w = getenv("LVSA_D64_WAVES");
  return a->D == 64 && a->block_q == kPPBM && a->dtype != LVSA_FP32 && !(w && strcmp(w, "8") == 0);
}

// Video tiles split in key-range halves at the end of each work queue, with
// the dual map: its two work-groups per CU take whole tiles at half the CU's
// rate, so a last round of whole tiles leaves CUs idle for longer.  As many
// per queue as the queue has work-groups on its XCD, halved (32), so that the
// last round runs half tiles, and at most the queue's video tiles
// (CogVideoX 0.9% faster; the 8-wave maps, one work-group per CU, gain
// nothing from it: Wan 4x and HunyuanVideo within +-0.5%).  0 for other maps,
// fp32, calls too small for the work queues, or with LVSA_VIDEO_SPLIT=0.
int vsplit_pref(const lvsa_attn_args* a) {
  const char* e = getenv("LVSA_VIDEO_SPLIT");
  if ((e && strcmp(e, "0") == 0) || !dual_map(a) || a->n_q == 0) return 0;
  const int per_cu = 2;
  const int64_t cus = cu_count();
  const int64_t vwork = ceil_div(a->n_q, a->block_q) * a->H * a->B;
  const int64_t work = vwork + ceil_div(a->n_tq, a->block_q) * text_chunks_of(a) * a->H * a->B;
  if (cus <= 0 || work <= per_cu * cus) return 0;
  const int64_t s = per_cu * cus / (2 * kXcds), per_queue = ceil_div(vwork, kXcds);
  return (int)(s < per_queue ? s : per_queue);
}

// Exact log-sum-exp merge of the text chunks (lvsa-vllm-omni/lvsa_vllm_omni/
// flashinfer_runner.py:184-197 merges two key sets the same way): with m_c the
// running max (log2 units), l_c the row sum and o_c the unnormalised O of
// chunk c, O = sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c, M = max_c m_c.
// One thread per 4 consecutive d of one (batch, head, text row).
template <typename E>
__global__ __launch_bounds__(256) void attn_text_merge_kernel(const float* ws, int chunks, int B, int H, int n_tq,
                                                              int D, char* ot, int64_t s0, int64_t s1, int64_t s2,
                                                              float* lse_t) {
  const int g4 = D / 4;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_bh = (int64_t)n_tq * g4;
  if (t >= per_bh * B * H) return;
  const int64_t bh = t / per_bh;
  const int row = (int)((t % per_bh) / g4), dq = (int)(t % g4);
  const int head = (int)(bh % H), batch = (int)(bh / H);
  const int64_t stride_c = (int64_t)B * H * n_tq;  // slots per chunk
  const int64_t slot0 = bh * n_tq + row;
  const float2* ml = reinterpret_cast<const float2*>(ws + text_ws_o_elems(chunks, B, H, n_tq, D));
  float M = -INFINITY;
  for (int c = 0; c < chunks; ++c) M = fmaxf(M, ml[c * stride_c + slot0].x);
  float L = 0.f;
  float4 acc = float4{0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < chunks; ++c) {
    const float2 mc = ml[c * stride_c + slot0];
    const float w = __builtin_amdgcn_exp2f(mc.x - M);
    const float4 o = *reinterpret_cast<const float4*>(ws + (c * stride_c + slot0) * D + 4 * dq);
    L += w * mc.y;
    acc.x += w * o.x;
    acc.y += w * o.y;
    acc.z += w * o.z;
    acc.w += w * o.w;
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  E* op = reinterpret_cast<E*>(ot + 2 * (batch * s0 + row * s1 + head * s2)) + 4 * dq;
  op[0] = (E)(acc.x * inv);
  op[1] = (E)(acc.y * inv);
  op[2] = (E)(acc.z * inv);
  op[3] = (E)(acc.w * inv);
  if (lse_t && dq == 0)
    lse_t[bh * n_tq + row] = L > 0.f ? (M + __log2f(L)) * 0.69314718055994530942f : -INFINITY;
}

// Merge of the two halves of the split video tiles (vsplit slots per queue):
// one thread per (slot, row, 4 columns), the exact log-sum-exp combination
// of attn_text_merge_kernel, written where the unsplit tile writes O and LSE.
template <typename E>
__global__ __launch_bounds__(256) void attn_video_merge_kernel(AttnParams p, int block_q, int D) {
  const int g4 = D / 4;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_slot = (int64_t)block_q * g4;
  const int64_t slot = t / per_slot;   // x * vsplit + s
  if (slot >= (int64_t)kXcds * p.vsplit) return;
  const int x = (int)(slot / p.vsplit), sx = (int)(slot % p.vsplit);
  const QueueShape q = queue_shape(p, x);
  if (sx >= q.n_split) return;
  const int w = q.v0 + q.n_video - q.n_split + sx;
  const int tile = w % p.n_vt, rest = w / p.n_vt, head = rest % p.H, batch = rest / p.H;
  const int r = (int)((t % per_slot) / g4), dq = (int)(t % g4);
  const int64_t row = (int64_t)tile * block_q + r;
  if (row >= p.n_q) return;
  const float2* ml = reinterpret_cast<const float2*>(p.vws + video_ws_o_elems(p.vsplit, block_q, D));
  const int64_t i0 = (2 * slot) * block_q + r, i1 = i0 + block_q;
  const float2 a0 = ml[i0], a1 = ml[i1];
  const float M = fmaxf(a0.x, a1.x);
  const float w0 = __builtin_amdgcn_exp2f(a0.x - M), w1 = __builtin_amdgcn_exp2f(a1.x - M);
  const float L = w0 * a0.y + w1 * a1.y;
  const float4 o0 = *reinterpret_cast<const float4*>(p.vws + i0 * D + 4 * dq);
  const float4 o1 = *reinterpret_cast<const float4*>(p.vws + i1 * D + 4 * dq);
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  E* op = reinterpret_cast<E*>(p.o + 2 * (batch * p.o_str[0] + row * p.o_str[1] + head * p.o_str[2])) + 4 * dq;
  op[0] = (E)((w0 * o0.x + w1 * o1.x) * inv);
  op[1] = (E)((w0 * o0.y + w1 * o1.y) * inv);
  op[2] = (E)((w0 * o0.z + w1 * o1.z) * inv);
  op[3] = (E)((w0 * o0.w + w1 * o1.w) * inv);
  if (p.lse && dq == 0)
    p.lse[((int64_t)batch * p.H + head) * p.n_q + row] =
        L > 0.f ? (M + __log2f(L)) * 0.69314718055994530942f : -INFINITY;
}

// Whether the short last key block of the frame-structured source crosses a
// frame boundary: it holds the t = n_k - 64 floor((n_k - 1) / 64) < 64 last
// keys, tokens [k_tok0 + n_k - t, k_tok0 + n_k), and the last boundary at or
// below its end lies e = (k_tok0 + n_k) mod C tokens before that end.  The
// plan builder describes such a block as "generic" (two frames and the rows
// past the end of the source).
bool stream_tail_crosses_frame(int64_t n_q, int64_t n_k, int64_t k_tok0, int C) {
  if (n_q == 0 || n_k <= 0 || C <= 0) return false;
  const int64_t t = n_k - kBN * ((n_k - 1) / kBN);
  const int64_t e = (k_tok0 + n_k) % C;
  return t < kBN && e > 0 && e < t;
}

bool aligned16(const void* ptr, const int64_t* str, int n, int elem_bytes) {
  if (((uintptr_t)ptr) % 16) return false;
  for (int i = 0; i < n; ++i)
    if ((str[i] * elem_bytes) % 16) return false;
  return true;
}

}  // namespace

extern "C" int lvsa_attn_fwd(const lvsa_attn_args* a, hipStream_t stream) {
  clear_error();
  LVSA_REQUIRE(a != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: null args");
  LVSA_REQUIRE(a->D == 64 || a->D == 96 || a->D == 128 || a->D == 192 || a->D == 256, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: head_dim %d not supported (64, 96, 128, 192, 256)", a->D);
  LVSA_REQUIRE(a->D < 192 || a->block_q == kBM || (a->D == 192 && a->block_q == kPPBM), LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: head_dim %d runs 128-row tiles (192 also 256-row ones; block_q %d)", a->D,
               a->block_q);
  LVSA_REQUIRE(a->dtype == LVSA_BF16 || a->dtype == LVSA_FP16 || a->dtype == LVSA_FP32, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: dtype %d", a->dtype);
  const bool fp32 = a->dtype == LVSA_FP32;
  const int es = fp32 ? 4 : 2;   // bytes per element
  LVSA_REQUIRE(fp32 || a->D != 96 || a->block_q == kPPBM, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: head_dim 96 runs 256-row tiles (block_q %d)", a->block_q);
  LVSA_REQUIRE(!fp32 || a->block_q == kBM, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: fp32 runs 128-row tiles (block_q %d)", a->block_q);
  LVSA_REQUIRE(a->B >= 1 && a->H >= 1 && a->Hkv >= 1 && a->H % a->Hkv == 0, LVSA_ERR_INVALID_ARG,
               "lvsa_attn_fwd: B=%d H=%d Hkv=%d (H must be a multiple of Hkv)", a->B, a->H, a->Hkv);
  LVSA_REQUIRE(a->n_q >= 0 && a->n_k >= 0 && a->n_x >= 0 && a->n_tq >= 0, LVSA_ERR_INVALID_ARG,
               "lvsa_attn_fwd: negative length");
  LVSA_REQUIRE(a->tile_indptr && a->entries, LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: missing plan");
  LVSA_REQUIRE(a->block_q == kBM || a->block_q == kPPBM || a->block_q == kStream12BM, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: block_q %d (the kernels tile 128, 256 or 384 query rows)", a->block_q);
  // 384-row tiles: the 12-wave single-stream kernel, head size 64 in 16 bit;
  // its loop handles descriptors "none" and "two-part" only, which is all a
  // plan holds when a tile touches at most two query frames (frames of at
  // least 383 rows) and a key block at most two key frames (at least 64).
  LVSA_REQUIRE(a->block_q != kStream12BM ||
                   (a->D == 64 && !fp32 && (a->n_q == 0 || (a->R >= kStream12BM - 1 && a->C >= kBN))),
               LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: 384-row tiles need head_dim 64 in bf16/fp16 and frames of >= 383 query and >= 64 "
               "key rows (head_dim %d, R %d, C %d); build the plan with block_q 256", a->D, a->R, a->C);
  const int n_vt = (int)ceil_div(a->n_q, a->block_q), n_tt = (int)ceil_div(a->n_tq, a->block_q);
  LVSA_REQUIRE(a->n_video_tiles == n_vt && a->n_tiles == n_vt + n_tt, LVSA_ERR_INVALID_ARG,
               "lvsa_attn_fwd: plan has %d/%d tiles, expected %d/%d for block_q %d", a->n_video_tiles,
               a->n_tiles, n_vt, n_vt + n_tt, a->block_q);
  LVSA_REQUIRE(a->n_q == 0 || (a->q && a->o), LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: null q/o");
  LVSA_REQUIRE(a->n_tq == 0 || (a->qt && a->ot), LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: null text q/o");
  LVSA_REQUIRE(a->n_k == 0 || (a->k && a->v), LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: null k/v");
  LVSA_REQUIRE(a->n_x == 0 || (a->kx && a->vx), LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: null extra k/v");
  LVSA_REQUIRE(a->n_k + a->n_x > 0 || a->n_tiles == 0, LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: no keys");
  bool ok = true;
  if (a->n_q) ok = ok && aligned16(a->q, a->q_str, 3, es) && aligned16(a->o, a->o_str, 3, es);
  if (a->n_tq) ok = ok && aligned16(a->qt, a->qt_str, 3, es) && aligned16(a->ot, a->ot_str, 3, es);
  if (a->n_k) ok = ok && aligned16(a->k, a->k_str, 3, es) && aligned16(a->v, a->v_str, 3, es);
  if (a->n_x) ok = ok && aligned16(a->kx, a->kx_str, 3, es) && aligned16(a->vx, a->vx_str, 3, es);
  LVSA_REQUIRE(ok, LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd: tensors must be 16-byte aligned with 16-byte row strides");
  // per-lane DMA offsets within a 64-row key block are 32-bit
  auto fits = [&](int64_t row_elems) { return row_elems >= 0 && row_elems * es * (kBN - 1) + es * (int64_t)a->D <= 0xFFFFFFFFLL; };
  LVSA_REQUIRE(fits(a->k_str[1]) && fits(a->v_str[1]) && (a->n_x == 0 || (fits(a->kx_str[1]) && fits(a->vx_str[1]))),
               LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd: key/value row stride too large");
  // the 256-row kernel forms per-lane row offsets with 24-bit multiplies
  auto fits24 = [&](int64_t row_elems) { return row_elems * 2 < (1LL << 24); };
  LVSA_REQUIRE(a->block_q == kBM || (fits24(a->k_str[1]) && fits24(a->v_str[1]) &&
                                       (a->n_x == 0 || (fits24(a->kx_str[1]) && fits24(a->vx_str[1])))),
               LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd: key/value row stride of 16 MiB or more (block_q %d)",
               a->block_q);
  // Every query row must have a relation row (generic blocks read it).
  if (a->n_q > 0) {
    const int64_t R = a->R > 0 ? a->R : 1;
    const int64_t first = a->q_tok0 / R - a->q_frame0, last = (a->q_tok0 + a->n_q - 1) / R - a->q_frame0;
    LVSA_REQUIRE(a->q_tok0 >= 0 && a->k_tok0 >= 0 && first >= 0 && last < a->rel_rows && a->rel && a->words >= 1,
                 LVSA_ERR_INVALID_ARG,
                 "lvsa_attn_fwd: query rows map to relation rows [%lld, %lld], the relation has %d rows",
                 (long long)first, (long long)last, a->rel_rows);
  }
  const int chunks = a->workspace ? text_chunks_of(a) : 1;
  const int64_t ws_need = a->workspace ? ws_bytes(a, 0) : 0;   // without the video split
  LVSA_REQUIRE(a->workspace_bytes >= ws_need, LVSA_ERR_CAPACITY,
               "lvsa_attn_fwd: workspace of %lld bytes < %lld needed (lvsa_attn_workspace_query)",
               (long long)a->workspace_bytes, (long long)ws_need);
  LVSA_REQUIRE(ws_need == 0 || ((uintptr_t)a->workspace) % 16 == 0, LVSA_ERR_INVALID_ARG,
               "lvsa_attn_fwd: workspace must be 16-byte aligned");
  const int64_t vwork = (int64_t)n_vt * a->H * a->B, twork = (int64_t)n_tt * chunks * a->H * a->B;
  const int64_t work = vwork + twork;
  LVSA_REQUIRE(work < (int64_t)INT32_MAX, LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: too much work");
  if (work == 0) return LVSA_OK;

  AttnParams p;
  p.q = (const char*)a->q;
  p.k = (const char*)a->k;
  p.v = (const char*)a->v;
  p.kx = (const char*)a->kx;
  p.vx = (const char*)a->vx;
  p.qt = (const char*)a->qt;
  p.o = (char*)a->o;
  p.ot = (char*)a->ot;
  p.lse = a->lse;
  p.lse_t = a->lse_t;
  for (int i = 0; i < 3; ++i) {
    p.q_str[i] = a->q_str[i];
    p.k_str[i] = a->k_str[i];
    p.v_str[i] = a->v_str[i];
    p.kx_str[i] = a->kx_str[i];
    p.vx_str[i] = a->vx_str[i];
    p.qt_str[i] = a->qt_str[i];
    p.o_str[i] = a->o_str[i];
    p.ot_str[i] = a->ot_str[i];
  }
  p.B = a->B;
  p.H = a->H;
  p.Hkv = a->Hkv;
  p.group = a->H / a->Hkv;
  p.n_q = a->n_q;
  p.n_k = a->n_k;
  p.n_x = a->n_x;
  p.n_tq = a->n_tq;
  p.scale_log2 = a->scale * 1.4426950408889634f;
  p.tile_indptr = a->tile_indptr;
  p.entries = reinterpret_cast<const uint2*>(a->entries);
  p.n_tiles = a->n_tiles;
  p.n_vt = n_vt;
  p.n_tt = n_tt;
  p.rel = a->rel;
  p.words = a->words;
  p.R = a->R > 0 ? a->R : 1;
  p.C = a->C > 0 ? a->C : 1;
  p.q_frame0 = a->q_frame0;
  p.q_tok0 = a->q_tok0;
  p.k_tok0 = a->k_tok0;
  p.total_work = (int)work;
  p.n_vwork = (int)vwork;
  p.n_twork = (int)twork;
  p.text_chunks = chunks;
  p.text_first = chunks == 1 ? 1 : 0;
  p.ws = chunks > 1 ? (float*)a->workspace : nullptr;
  p.vsplit = 0;
  p.vws = nullptr;
  // The single-stream kernel (D = 64, 96 and 128 here; 192 and 256 below)
  // serves plans without generic descriptors:
  // 256-row tiles touch at most two query frames when frames have >= 255
  // rows, and 64-key blocks (even short last ones) at most two key frames
  // when frames have >= 64 keys.  LVSA_ATTN_KERNEL=pp selects the ping-pong
  // kernel instead (comparisons).
  const char* kenv = getenv("LVSA_ATTN_KERNEL");
  const bool force_pp = kenv != nullptr && strcmp(kenv, "pp") == 0;
  // Its copies address a whole key source through one buffer resource with
  // 32-bit byte offsets; at D = 96 and 192 the lanes of the unused chunks of
  // a row add 0x7FFF0000 to theirs, which must lie past the end of the
  // source (zeros, no access) or inside it (a harmless read into chunks no
  // read touches): the rows must stay below 2^31 bytes there.
  const int64_t lim = (a->D == 96 || a->D == 192) ? (1LL << 31) : (1LL << 32);
  auto fits32 = [lim](int64_t rows, int64_t row_elems) { return (rows + kBN) * row_elems * 2 < lim; };
  const bool src32 = fits32(a->n_k, a->k_str[1]) && fits32(a->n_k, a->v_str[1]) &&
                     (a->n_x == 0 || (fits32(a->n_x, a->kx_str[1]) && fits32(a->n_x, a->vx_str[1])));
  // Its lane copy offsets are 24-bit products (row x row stride in bytes).
  const bool str24 = fits24(a->k_str[1]) && fits24(a->v_str[1]) &&
                     (a->n_x == 0 || (fits24(a->kx_str[1]) && fits24(a->vx_str[1])));
  // Its loop masks "two-part" descriptors only.  A short last key block of
  // the frame source that crosses a frame boundary (a source starting
  // mid-frame, as on a context-parallel shard) has three parts (two frames
  // and the rows past the end) and is planned "generic".
  const bool tail_cross = stream_tail_crosses_frame(a->n_q, a->n_k, a->k_tok0, p.C);
  const bool stream_src = src32 && str24 && !tail_cross;
  p.use_stream = (!fp32 && (a->D == 128 || a->D == 96 || a->D == 64) && a->block_q == kPPBM && !force_pp &&
                  stream_src && (a->n_q == 0 || (p.R >= 255 && p.C >= 64))) ? 1 : 0;
  // D = 192 and 256: the wide single-stream loop on the 4-wave kernel's
  // 128-row tiles, which touch at most two query frames when frames have
  // >= 127 rows.
  if (!fp32 && (a->D == 192 || a->D == 256) && a->block_q == kBM && !force_pp && stream_src &&
      (a->n_q == 0 || (p.R >= 127 && p.C >= 64)))
    p.use_stream = 1;
  // D = 192 on 256-row tiles: the loop's dual-wide map, the only kernel for
  // them (frames of >= 255 query rows).
  if (a->D == 192 && a->block_q == kPPBM) {
    LVSA_REQUIRE(!force_pp && stream_src && (a->n_q == 0 || (p.R >= 255 && p.C >= 64)), LVSA_ERR_UNSUPPORTED,
                 "lvsa_attn_fwd: head_dim 192 on 256-row tiles needs frames of >= 255 query and >= 64 key rows, "
                 "key sources below 2^31 bytes with row strides below 16 MiB, the last key block of the frame "
                 "source inside one frame, and no LVSA_ATTN_KERNEL=pp (R %d, C %d); build the plan with block_q 128",
                 p.R, p.C);
    p.use_stream = 1;
  }
  if (a->block_q == kStream12BM) {
    LVSA_REQUIRE(src32, LVSA_ERR_UNSUPPORTED,
                 "lvsa_attn_fwd: 384-row tiles address each key source with 32-bit byte offsets (source too large); "
                 "build the plan with block_q 256");
    LVSA_REQUIRE(!tail_cross, LVSA_ERR_UNSUPPORTED,
                 "lvsa_attn_fwd: 384-row tiles need the last key block of the frame source inside one frame "
                 "(n_k %lld, k_tok0 %lld, C %d); build the plan with block_q 256",
                 (long long)a->n_k, (long long)a->k_tok0, p.C);
    p.use_stream = 1;
  }
  // D = 64 on 256-row tiles: the dual map (64 rows per wave, 4 waves, two
  // work-groups per CU); LVSA_D64_WAVES=8 selects 8 waves of 32 rows instead
  // (comparisons).
  p.dual = (p.use_stream && dual_map(a)) ? 1 : 0;
  // With a workspace, the single-stream kernel runs one persistent
  // work-group per CU (two with the dual map) over the work queues (counters
  // zeroed first).
  p.queues = nullptr;
  p.grid = (int)work;
  const int cus = cu_count();
  const int per_cu = p.dual ? 2 : 1;
  if (p.use_stream && a->workspace && cus > 0 && work > per_cu * cus) {
    // the video split when the workspace holds its partials (the size
    // lvsa_attn_workspace_query returns), none otherwise
    const int vs = vsplit_pref(a);
    if (vs > 0 && a->workspace_bytes >= ws_bytes(a, vs)) {
      p.vsplit = vs;
      p.vws = (float*)((char*)a->workspace + video_offset(a, chunks));
    }
    p.queues = (uint32_t*)((char*)a->workspace + queue_offset(a, chunks, p.vsplit));
    p.grid = per_cu * cus;
    hipLaunchKernelGGL(queue_reset_kernel, dim3(1), dim3(64), 0, stream, p.queues);
    const int qrc = launch_status("lvsa_attn_fwd (queue reset)");
    if (qrc != LVSA_OK) return qrc;
  }
  const int bq = a->block_q;
  const bool bf16 = a->dtype == LVSA_BF16;
  int rc;
  if (fp32) rc = launch_f32(p, a->D, stream);
  else if (a->D == 256) rc = launch_d256(p, bq, bf16, stream);
  else if (a->D == 128) rc = launch_d128(p, bq, bf16, stream);
  else if (a->D == 96) rc = launch_d96(p, bq, bf16, stream);
  else if (a->D == 192) rc = launch_d192(p, bq, bf16, stream);
  else rc = launch_d64(p, bq, bf16, stream);
  if (rc != LVSA_OK) return rc;
  if (p.vsplit > 0) {
    const int64_t threads = (int64_t)kXcds * p.vsplit * bq * (a->D / 4);
    const dim3 grid((unsigned)ceil_div(threads, 256));
    if (bf16) hipLaunchKernelGGL(attn_video_merge_kernel<__bf16>, grid, dim3(256), 0, stream, p, bq, a->D);
    else hipLaunchKernelGGL(attn_video_merge_kernel<_Float16>, grid, dim3(256), 0, stream, p, bq, a->D);
    rc = launch_status("lvsa_attn_fwd (video merge)");
    if (rc != LVSA_OK) return rc;
  }
  if (chunks == 1) return rc;
  const int64_t threads = (int64_t)a->B * a->H * a->n_tq * (a->D / 4);
  const dim3 grid((unsigned)ceil_div(threads, 256));
  if (bf16) {
    hipLaunchKernelGGL(attn_text_merge_kernel<__bf16>, grid, dim3(256), 0, stream, (const float*)a->workspace,
                       chunks, a->B, a->H, a->n_tq, a->D, (char*)a->ot, a->ot_str[0], a->ot_str[1], a->ot_str[2],
                       a->lse_t);
  } else {
    hipLaunchKernelGGL(attn_text_merge_kernel<_Float16>, grid, dim3(256), 0, stream, (const float*)a->workspace,
                       chunks, a->B, a->H, a->n_tq, a->D, (char*)a->ot, a->ot_str[0], a->ot_str[1], a->ot_str[2],
                       a->lse_t);
  }
  return launch_status("lvsa_attn_fwd (text merge)");
}

namespace lvsa {
int64_t attn_workspace_min_bytes(const lvsa_attn_args* a) { return ws_bytes(a, 0); }
}  // namespace lvsa

extern "C" int lvsa_attn_workspace_query(const lvsa_attn_args* a, int64_t* bytes) {
  clear_error();
  LVSA_REQUIRE(a != nullptr && bytes != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_attn_workspace_query: null pointer");
  LVSA_REQUIRE(a->n_k >= 0 && a->n_x >= 0 && a->n_tq >= 0 && a->B >= 1 && a->H >= 1, LVSA_ERR_INVALID_ARG,
               "lvsa_attn_workspace_query: bad sizes");
  LVSA_REQUIRE(a->D == 64 || a->D == 96 || a->D == 128 || a->D == 192 || a->D == 256, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_workspace_query: head_dim %d not supported", a->D);
  *bytes = ws_bytes(a, vsplit_pref(a));
  return LVSA_OK;
}
