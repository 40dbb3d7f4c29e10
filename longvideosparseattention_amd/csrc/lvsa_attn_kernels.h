// Compiler-built kernels of the block-sparse attention forward (gfx950) and
// what they share with the hand-scheduled single-stream kernel
// (lvsa_attn_stream.h): parameters, plan entries, work queues, the text
// split.  One translation unit per head size instantiates them
// (lvsa_attn_d{64,96,128,192,256}.hip, each with the machine scheduler
// measured fastest for it; lvsa_attn.hip holds the C ABI).
//
// Two kernels here walk the key blocks (BN = 64 rows each) that the block
// plan lists for a query tile of one head; they serve the geometries the
// single-stream kernel does not take (frames too short for it) and the
// LVSA_ATTN_KERNEL=pp comparison:
//   attn_fwd_pp_kernel   256-row tiles, 8 waves x 32 rows in two groups that
//                        alternate an MFMA phase with a softmax phase (D = 64,
//                        96 and 128);
//   attn_fwd_kernel      128-row tiles, 4 waves x 32 rows, one barrier per
//                        block (D = 192 and 256, whose Q and O need 320
//                        registers; any head size with LVSA_ATTN_BLOCK_Q=128).
// Both compute, per wave and key block:
//   S^T = K · Q^T      v_mfma_f32_32x32x16_{bf16,f16}: A = K rows from LDS
//                      (ds_read_b128), B = Q held in registers for the tile
//   softmax            every lane owns one query row (column of S^T): 16 of
//                      the 32 keys of a 32-key sub-tile, the other 16 sit in
//                      lane ^ 32; the running max uses a lazy rescale (O and
//                      the row sum are rescaled only when the block maximum
//                      exceeds the running one by more than 2^8)
//   O^T += V^T · P^T   A = V^T read from the row-major LDS tile with
//                      ds_read_b64_tr_b16, B = P (bf16/f16) straight from the
//                      S^T accumulator registers (key order permuted
//                      identically on both operands)
//
// K and V blocks are copied global -> LDS without a VGPR round trip (the
// 4-wave kernel: global_load_lds_dwordx4 into a double buffer; the ping-pong
// kernel: buffer_load_dwordx4 ... lds into a 4-stage ring), with a
// 16-byte-chunk XOR swizzle that keeps both the K reads and the transposing V
// reads free of bank conflicts.  The LDS image of a block is row-major, so K
// and V are read in place from the caller's [B, S, H, D] tensors: no gather,
// no transpose, no padding copies.
#pragma once
#include "lvsa_common.h"

#include <type_traits>

namespace lvsa {

struct AttnParams {
  const char* q;
  const char* k;
  const char* v;
  const char* kx;
  const char* vx;
  const char* qt;
  char* o;
  char* ot;
  float* lse;
  float* lse_t;
  int64_t q_str[3], k_str[3], v_str[3], kx_str[3], vx_str[3], qt_str[3], o_str[3], ot_str[3];
  int B, H, Hkv, group;
  int n_q, n_k, n_x, n_tq;
  float scale_log2;
  const int32_t* tile_indptr;
  const uint2* entries;
  int n_tiles, n_vt, n_tt;
  const uint32_t* rel;
  int words, R, C, q_frame0;
  int64_t q_tok0, k_tok0;
  int total_work;
  // Work items: n_vwork video tiles (n_vt per head) and n_twork text items
  // (n_tt tiles per head, each split into text_chunks key ranges).  Unsplit
  // text tiles (text_chunks == 1) are the longest items and go first; split
  // ones go last, where their chunks fill the launch's final round, and write
  // unnormalised partials to ws for attn_text_merge_kernel.
  int n_vwork, n_twork, text_chunks, text_first;
  float* ws;
  // D = 128, 256-row tiles: run the single-stream kernel (its loop handles
  // descriptors "none" and "two-part", which is all such a plan holds when
  // query frames span at least 255 rows and key frames at least 64)
  int use_stream;
  // D = 64, 256-row tiles on the single-stream kernel: the dual map (4 waves
  // of 64 rows, two work-groups per CU) rather than 8 waves of 32 rows
  int dual;
  // Key-range split of each queue's last video tiles (with the work queues):
  // the last min(vsplit, videos of the queue) video items of queue x run as
  // two halves of their entry lists, after the queue's whole tiles, and write
  // unnormalised partials to slots x * vsplit + s of vws (fp32 O [slot][half]
  // [block_q][D], then (running max, row sum) [slot][half][block_q]) for
  // attn_video_merge_kernel.  0: no split.
  int vsplit;
  float* vws;
  // Work queues (single-stream kernel with a workspace): `grid` persistent
  // work-groups, one per CU (two with the dual map), take work items from 8 queues, one per XCD,
  // whose counters (kQueueStride bytes apart, zeroed before the launch) are
  // at `queues`; null: one work-group per item, mapped by map_work.
  uint32_t* queues;
  int grid;
};

// Bytes of the work-queue counters at the end of the attention workspace.
constexpr int kQueueStride = 128;                  // one counter per 128-byte line
constexpr int64_t kQueueBytes = 8 * kQueueStride;

// Layout of the text-split scratch: O partials [chunk][B][H][n_tq][D] fp32,
// then (running max in log2 units, row sum) pairs [chunk][B][H][n_tq].
__host__ __device__ inline int64_t text_ws_o_elems(int chunks, int B, int H, int n_tq, int D) {
  return (int64_t)chunks * B * H * n_tq * D;
}

// Launches per head size (bf16 / fp16), each compiled in its own translation
// unit (lvsa_attn_d<D>.hip): the compiler's code for one head size then does
// not depend on which others are instantiated beside it, and each unit takes
// the machine scheduler measured best for it.
int launch_d64(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream);
int launch_d96(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream);
int launch_d128(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream);
int launch_d192(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream);
int launch_d256(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream);
// fp32 inputs (lvsa_attn_f32.hip): 128-row tiles, every head size.
int launch_f32(const AttnParams& prm, int D, hipStream_t stream);

namespace {

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kXcds = 8;

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;


template <typename E>
struct Ops;

template <>
struct Ops<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  __device__ static floatx16 mfma(v8 a, v8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static v2 pack(float a, float b) { return v2{(__bf16)a, (__bf16)b}; }
  __device__ static float dot2(v2 a, float acc) {
    const v2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(a, one, acc, false);
  }
  __device__ static unsigned short bits(float x) { return __builtin_bit_cast(unsigned short, (__bf16)x); }
  __device__ static v8 scale(v8 x, float a) {
    v8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)((float)x[i] * a);
    return r;
  }
};

template <>
struct Ops<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  __device__ static floatx16 mfma(v8 a, v8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static v2 pack(float a, float b) { return v2{(_Float16)a, (_Float16)b}; }
  __device__ static float dot2(v2 a, float acc) {
    const v2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(a, one, acc, false);
  }
  __device__ static unsigned short bits(float x) { return __builtin_bit_cast(unsigned short, (_Float16)x); }
  __device__ static v8 scale(v8 x, float a) {
    v8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)((float)x[i] * a);
    return r;
  }
};

// 16-byte-chunk swizzle of LDS row r (r & 15 is all that matters).
//  D = 128, and D = 96 laid out on the same 256-byte row pitch (chunks 12-15
//    of a D = 96 row hold zeros and are never read)
//    (16 chunks/row, a row spans all 64 banks): a bijection on r & 15 so
//    the 16 rows of a K read hit 16 distinct chunks, and bits 2-3 = r & 3 so
//    the 4 rows of a transposing V read land in 4 distinct 64-byte quarters.
//  D = 64 (8 chunks/row, 2 rows per bank line): a bijection on (r >> 1) & 7
//    with bit 2 = (r >> 1) & 1 so rows r and r + 2 of a V read differ.
//  D = 256, and D = 192 laid out on the same 512-byte row pitch (chunks 24-31
//    of a D = 192 row are never read) (32 chunks/row, a row spans the banks
//    twice): the D = 128 swizzle on the low 4 chunk bits, which keeps both
//    patterns inside one 256-byte half.
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D == 96 || D == 128 || D == 192 || D == 256) {
    return ((r & 3) << 2) | ((r >> 2) & 3);
  } else {
    return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
  }
}

__device__ __forceinline__ void dma16(const void* g, lds_char* l) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

// The same copy issued as inline asm.  The compiler does not see the LDS
// write, so it inserts no vmcnt wait before later LDS reads it cannot prove
// disjoint (it cannot for the ring stages, and such a wait makes every copy
// synchronous); the kernel orders the copies itself with explicit vmcnt
// waits and barriers.  The addresses are made uniform so both land in SGPRs;
// the s_nop covers the M0-write -> LDS-DMA hazard.  Nothing else in a kernel
// that uses this may rely on M0.
__device__ __forceinline__ void dma16_async(const char* g, uint32_t voff, const lds_char* l) {
  // readfirstlane returns int: go through uint32_t so nothing sign-extends
  const uint64_t b = (uint64_t)g;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
  const uint32_t la = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)l);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sb), "s"(la) : "m0");
#pragma clang diagnostic pop
}

// 16 bytes per lane, global -> LDS, through a buffer resource: lanes whose
// soffset + voffset + 16 exceed the resource's num_records read zeros (per
// dword) and write them to LDS, with no memory access.  Issued as asm for
// the same reason as dma16_async.
__device__ __forceinline__ void dma16_buf(u32x4 rsrc, uint32_t voff, uint32_t soff, const lds_char* l) {
  const uint32_t la = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)l);
  const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane((int)soff);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" : : "v"(voff), "s"(rsrc), "s"(so), "s"(la) : "m0");
#pragma clang diagnostic pop
}

__device__ __forceinline__ void wait_vm0() {
  // s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

// The work item of this work-group.  Video tiles are remapped so that
// consecutive tiles of one head run on one XCD (work-groups are dispatched to
// the 8 XCDs round-robin, and each XCD has its own L2): XCD x takes a
// contiguous range of the video items.  Text items keep the dispatch order.
struct WorkItem {
  int tile, head, batch, chunk;
  bool text;
  int vhalf, vslot;   // a split video tile: half 0 or 1 and its partial slot; vhalf -1: whole
};
__device__ __forceinline__ WorkItem map_work(const AttnParams& p) {
  WorkItem it;
  const int b = blockIdx.x;
  const int tb0 = p.text_first ? 0 : p.n_vwork;  // first block of the text items
  const int vb0 = p.text_first ? p.n_twork : 0;  // first block of the video items
  if (b >= tb0 && b < tb0 + p.n_twork) {
    int t = b - tb0;
    it.chunk = t % p.text_chunks;
    t /= p.text_chunks;
    it.tile = p.n_vt + t % p.n_tt;
    t /= p.n_tt;
    it.head = t % p.H;
    it.batch = t / p.H;
    it.text = true;
    it.vhalf = -1;
    it.vslot = 0;
    return it;
  }
  const int x = b % kXcds;
  const int per = p.n_vwork / kXcds, rem = p.n_vwork % kXcds;
  // video items on XCD y: per, plus one for the first `rem` XCDs in dispatch
  // order after block vb0
  int start = 0;
  for (int y = 0; y < x; ++y) start += per + ((((y - vb0) % kXcds + kXcds) % kXcds) < rem ? 1 : 0);
  const int first = vb0 + (((x - vb0) % kXcds + kXcds) % kXcds);  // first video block on XCD x
  const int w = start + (b - first) / kXcds;
  it.tile = w % p.n_vt;
  const int rest = w / p.n_vt;
  it.head = rest % p.H;
  it.batch = rest / p.H;
  it.chunk = 0;
  it.text = false;
  it.vhalf = -1;
  it.vslot = 0;
  return it;
}

// Work queues.  Queue x (one per XCD) holds, in this order: the unsplit text
// items t = x, x + 8, ... (the longest, first), the video items of the same
// XCD-contiguous range map_work gives XCD x (consecutive tiles of a head, so
// the K/V blocks they share stay in that XCD's L2), the last n_split of them
// as two halves each (key-range halves of their entry lists), and the split
// text chunks t = x, x + 8, ... (the shortest, last).  The halves and the
// chunks make the launch's last round finer than whole tiles.  A work-group takes items from the
// queue of its own XCD and, once that is empty, from the next ones in turn:
// XCDs that run faster take over the items of the slower ones at the end, so
// the launch does not wait for the slowest XCD's fixed share.
struct QueueShape {
  int n_first, v0, n_video, n_split, n_last;   // n_split of the n_video video items run as two halves
};
__host__ __device__ inline QueueShape queue_shape(const AttnParams& p, int x) {
  QueueShape q;
  const int first = p.text_first ? p.n_twork : 0, last = p.text_first ? 0 : p.n_twork;
  q.n_first = (first - x + kXcds - 1) / kXcds;   // items x, x + 8, ... below `first` (x < 8)
  q.n_last = (last - x + kXcds - 1) / kXcds;
  const int per = p.n_vwork / kXcds, rem = p.n_vwork % kXcds;
  q.v0 = x * per + (x < rem ? x : rem);
  q.n_video = per + (x < rem ? 1 : 0);
  q.n_split = p.vsplit < q.n_video ? p.vsplit : q.n_video;
  return q;
}

// Items in queue x.
__host__ __device__ inline int queue_items(const QueueShape& q) { return q.n_first + q.n_video + q.n_split + q.n_last; }

__host__ __device__ inline WorkItem text_item(const AttnParams& p, int t) {
  WorkItem it;
  it.chunk = t % p.text_chunks;
  t /= p.text_chunks;
  it.tile = p.n_vt + t % p.n_tt;
  t /= p.n_tt;
  it.head = t % p.H;
  it.batch = t / p.H;
  it.text = true;
  it.vhalf = -1;
  it.vslot = 0;
  return it;
}

// Item j of queue x.
__host__ __device__ inline WorkItem queue_item(const AttnParams& p, int x, int j) {
  const QueueShape q = queue_shape(p, x);
  if (j < q.n_first) return text_item(p, x + kXcds * j);
  j -= q.n_first;
  const int n_whole = q.n_video - q.n_split;
  if (j >= n_whole + 2 * q.n_split) return text_item(p, x + kXcds * (j - n_whole - 2 * q.n_split));
  WorkItem it;
  it.vhalf = -1;
  it.vslot = 0;
  int w = q.v0 + j;
  if (j >= n_whole) {                 // half j & 1 of split tile s of the queue
    const int s = (j - n_whole) >> 1;
    w = q.v0 + n_whole + s;
    it.vhalf = (j - n_whole) & 1;
    it.vslot = x * p.vsplit + s;
  }
  it.tile = w % p.n_vt;
  const int rest = w / p.n_vt;
  it.head = rest % p.H;
  it.batch = rest / p.H;
  it.chunk = 0;
  it.text = false;
  return it;
}

// Next item for the calling work-group (one thread calls it): (j << 3) | x
// for item j of queue x, or -1 once every queue is empty.  `x` is the queue
// being drained and `dry` counts the queues found empty; counters only grow,
// so a queue found empty is not visited again and a work-group gives up after
// at most 8 failed increments.
__device__ __forceinline__ int queue_next(const AttnParams& p, int& x, int& dry) {
  while (dry < kXcds) {
    const QueueShape q = queue_shape(p, x);
    const uint32_t j = atomicAdd(p.queues + x * (kQueueStride / 4), 1u);
    if (j < (uint32_t)queue_items(q)) return (int)(j << 3) | x;
    x = (x + 1) & (kXcds - 1);
    ++dry;
  }
  return -1;
}

// XCD of the calling wave (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ int xcd_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & (kXcds - 1); }

// Epilogue of a text chunk: the unnormalised O row of this lane (d = 32*dt +
// 8*rq + 4*h .. +3 in oacc[dt][4*rq ..]) to `wo` (fp32), and the (running
// max, row sum) pair to `ml`, in the scratch layout of text_ws_o_elems.
template <int NT>
__device__ __forceinline__ void store_text_partial(char* wo, float* ml, int h, const floatx16* oacc, float m_run,
                                                   float l_tot) {
#pragma unroll
  for (int dt = 0; dt < NT; ++dt) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = 32 * dt + 8 * rq + 4 * h;
      *reinterpret_cast<float4*>(wo + 4 * d0) =
          float4{oacc[dt][4 * rq], oacc[dt][4 * rq + 1], oacc[dt][4 * rq + 2], oacc[dt][4 * rq + 3]};
    }
  }
  if (h == 0) *reinterpret_cast<float2*>(ml) = float2{m_run, l_tot};
}

// Elements of the O partials of the video split: vsplit slots per queue, two
// halves per slot, block_q rows of D.
__host__ __device__ inline int64_t video_ws_o_elems(int vsplit, int block_q, int D) {
  return (int64_t)kXcds * vsplit * 2 * block_q * D;
}

// A half of a split video tile writes its partials where a tile writes its
// output: row base, row stride and LSE pointer redirected to its slot, offset
// so that the tile's first row r0 lands on the slot's row 0.
template <int D>
__device__ __forceinline__ void video_partial_dst(const AttnParams& p, const WorkItem& it, int block_q, int64_t r0,
                                                  char*& obase, int64_t& ors, float*& lse) {
  const int64_t slot = 2 * (int64_t)it.vslot + it.vhalf;
  const uintptr_t ws = reinterpret_cast<uintptr_t>(p.vws);
  ors = 4 * D;
  obase = reinterpret_cast<char*>(ws + 4 * (slot * block_q - r0) * D);
  lse = reinterpret_cast<float*>(ws + 4 * (video_ws_o_elems(p.vsplit, block_q, D) + 2 * (slot * block_q - r0)));
}

// A split text item writes its partials where a tile writes its output: the
// row base, row stride and LSE pointer of the text branch are redirected to
// the scratch slots of (chunk, batch, head) (no extra state stays live
// through the key loop).
template <int D>
__device__ __forceinline__ void text_partial_dst(const AttnParams& p, const WorkItem& it, char*& obase,
                                                 int64_t& ors, float*& lse) {
  const int64_t slot = (((int64_t)it.chunk * p.B + it.batch) * p.H + it.head) * p.n_tq;
  obase = reinterpret_cast<char*>(p.ws + slot * D);
  ors = 4 * D;
  lse = p.ws + text_ws_o_elems(p.text_chunks, p.B, p.H, p.n_tq, D) + 2 * slot;
}

// Entry range [e0, e1) of the work item: the tile's plan entries, chunk
// `chunk` of text_chunks equal parts of them, or half `vhalf` of a split
// video tile's (the first half takes the odd entry).
__device__ __forceinline__ void item_entries(const AttnParams& p, const WorkItem& it, int& e0, int& e1) {
  e0 = p.tile_indptr[it.tile];
  e1 = p.tile_indptr[it.tile + 1];
  if (it.vhalf >= 0) {
    const int mid = e0 + (e1 - e0 + 1) / 2;
    if (it.vhalf == 0) e1 = mid;
    else e0 = mid;
  } else if (it.text && p.text_chunks > 1) {
    const int len = (e1 - e0 + p.text_chunks - 1) / p.text_chunks;
    const int a = e0 + it.chunk * len;
    e0 = a < e1 ? a : e1;
    e1 = e0 + len < e1 ? e0 + len : e1;
  }
}

// Mask of one key block for this lane's query row (row `tile_row` of its
// tile, `my_row` of its source), for a block of kind two-part or generic:
// bit r covers register r%16 of the S^T accumulator of key half r/16, which
// holds key 8q + j + 4h of the block with q = r/4, j = r%4 (h = lane / 32).
__device__ __forceinline__ uint32_t block_keep_bits(const AttnParams& p, uint32_t cx, uint32_t cy, int tile_row,
                                                    int64_t my_row, int nrows, int h) {
  if ((cy & 3u) == kKindTwoPart) {
    const int bits = (cy >> 2) & 0xF;
    const int kb = (int)((cy >> 8) & 0xFF) - 4 * h;
    const int qs = (cy >> 16) & 0xFF;
    const bool rb = tile_row >= qs;
    const uint32_t lo_ok = (bits >> (rb ? 2 : 0)) & 1;
    const uint32_t hi_ok = (bits >> (rb ? 3 : 1)) & 1;
    int n_lo = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = kb - 8 * q;
      n_lo += c < 0 ? 0 : (c > 4 ? 4 : c);
    }
    const uint32_t lo_mask = n_lo >= 32 ? 0xFFFFFFFFu : ((1u << n_lo) - 1u);
    return (lo_ok ? lo_mask : 0u) | (hi_ok ? ~lo_mask : 0u);
  }
  const bool extra = (cx >> 31) != 0;
  const int64_t k0 = (int64_t)(cx & 0x7fffffffu) * kBN;
  const int64_t nsrc = extra ? p.n_x : p.n_k;
  const int64_t qtok = p.q_tok0 + (my_row < nrows ? my_row : (int64_t)nrows - 1);
  const int qf_row = (int)(qtok / p.R) - p.q_frame0;
  const uint32_t* relrow = p.rel + (int64_t)qf_row * p.words;
  uint32_t keep = 0;
  for (int r = 0; r < 32; ++r) {
    const int64_t key = k0 + 8 * (r >> 2) + 4 * h + (r & 3);
    if (key < nsrc) {
      const int64_t kf = (p.k_tok0 + key) / p.C;
      if ((kf >> 5) < p.words && ((relrow[kf >> 5] >> (kf & 31)) & 1u)) keep |= 1u << r;
    }
  }
  return keep;
}

template <int D, typename E>
// Two work-groups per CU, except at D = 192 and 256 (their O and Q fragments
// alone take up to 192 registers per lane, and a 128 KiB LDS ring leaves room
// for one work-group): one work-group, registers up to 512.
__global__ __launch_bounds__(kThreads, D >= 192 ? 1 : 2) void attn_fwd_kernel(AttnParams p) {
  using O = Ops<E>;
  using v8 = typename O::v8;
  using v2 = typename O::v2;
  constexpr int RB = (D == 192 ? 256 : D) * 2;  // bytes per K/V row in LDS (D = 192: the D = 256 pitch)
  constexpr int NCH = RB / 16;            // 16-byte chunks per LDS row
  constexpr int NCV = D / 8;              // of which hold data
  constexpr int TILE = kBN * RB;          // bytes of one K or V block
  constexpr int STAGE = 2 * TILE;         // K block + V block
  constexpr int NI = TILE / 1024;         // 1 KiB DMA instructions per block
  constexpr int NIW = NI / kWaves;        // per wave
  constexpr int ND = D / 16;              // MFMA k-steps of S
  constexpr int NT = D / 32;              // 32-wide d tiles of O
  constexpr int RPI = 1024 / RB;          // block rows per DMA instruction
  static_assert(NI % kWaves == 0, "tile must split evenly over waves");

  __shared__ __attribute__((aligned(1024))) char smem_raw[2 * STAGE];
  lds_char* smem = (lds_char*)smem_raw;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;        // half of the wave
  const int i32 = lane & 31;      // query row of this lane within the wave

  const WorkItem it = map_work(p);
  const int tile = it.tile, head = it.head, batch = it.batch;
  const bool text = it.text;
  const int hk = head / p.group;

  const char* qbase;
  char* obase;
  int64_t qrs, ors;
  int nrows;
  int64_t r0;
  float* lse;
  if (!text) {
    qbase = p.q + 2 * (batch * p.q_str[0] + head * p.q_str[2]);
    obase = p.o + 2 * (batch * p.o_str[0] + head * p.o_str[2]);
    qrs = 2 * p.q_str[1];
    ors = 2 * p.o_str[1];
    nrows = p.n_q;
    r0 = (int64_t)tile * kBM;
    lse = p.lse ? p.lse + ((int64_t)batch * p.H + head) * p.n_q : nullptr;
  } else {
    qbase = p.qt + 2 * (batch * p.qt_str[0] + head * p.qt_str[2]);
    obase = p.ot + 2 * (batch * p.ot_str[0] + head * p.ot_str[2]);
    qrs = 2 * p.qt_str[1];
    ors = 2 * p.ot_str[1];
    nrows = p.n_tq;
    r0 = (int64_t)(tile - p.n_vt) * kBM;
    lse = p.lse_t ? p.lse_t + ((int64_t)batch * p.H + head) * p.n_tq : nullptr;
    if (p.text_chunks > 1) text_partial_dst<D>(p, it, obase, ors, lse);
  }
  const bool partial = text && p.text_chunks > 1;
  int e0, e1;
  item_entries(p, it, e0, e1);

  // Key sources: 0 = frame-structured key/value, 1 = dense extra rows.
  const char* kb0 = p.k + 2 * (batch * p.k_str[0] + hk * p.k_str[2]);
  const char* vb0 = p.v + 2 * (batch * p.v_str[0] + hk * p.v_str[2]);
  const char* kb1 = p.n_x ? p.kx + 2 * (batch * p.kx_str[0] + hk * p.kx_str[2]) : kb0;
  const char* vb1 = p.n_x ? p.vx + 2 * (batch * p.vx_str[0] + hk * p.vx_str[2]) : vb0;
  const uint32_t krs0 = (uint32_t)(2 * p.k_str[1]), vrs0 = (uint32_t)(2 * p.v_str[1]);
  const uint32_t krs1 = (uint32_t)(2 * p.kx_str[1]), vrs1 = (uint32_t)(2 * p.vx_str[1]);

  // DMA geometry: instruction ii of this wave fills LDS bytes
  // [(wave*NIW + ii) KiB, +1 KiB), i.e. block rows RPI*(wave*NIW + ii) + lane/NCH,
  // physical chunk lane%NCH.  Because wave*NIW is a multiple of 4 (D=128) or
  // 2 (D=64), the swizzle of those rows is  dma_c ^ ii  with a per-lane dma_c.
  // (D = 256: two rows per instruction, the swizzle of instruction ii's
  // rows is formed per instruction.)
  const uint32_t dma_lr = (uint32_t)(lane / NCH);
  uint32_t dma_c16;
  if constexpr (D == 128) {
    dma_c16 = (uint32_t)(((lane & 15) ^ ((lane >> 4) << 2)) * 16);
  } else if constexpr (D == 64) {
    dma_c16 = (uint32_t)(((lane & 7) ^ ((((lane >> 4) & 1) << 2) | (((lane >> 5) & 1) << 1))) * 16);
  } else {
    dma_c16 = 0;
  }
  auto c16_of = [&](int ii) __attribute__((always_inline)) {
    if constexpr (D >= 192) {
      const uint32_t row = (uint32_t)(RPI * (wave * NIW + ii)) + dma_lr;
      int c = (lane % NCH) ^ swz<D>((int)(row & 15));
      // D = 192: a slot past the row's data is never read; it copies a data
      // chunk of the same row, so every address stays inside the row
      if constexpr (NCV < NCH) c = c >= NCV ? c - (NCH - NCV) : c;
      return (uint32_t)(c * 16);
    } else {
      return dma_c16 ^ (uint32_t)(16 * (ii & (D == 128 ? 3 : 1)));
    }
  };

  // Plan entries of this tile, 64 at a time in a VGPR (lane i holds entry
  // base + i); a uniform entry is read with v_readlane.  The next batch is
  // prefetched one batch ahead so a batch switch never waits on memory.
  uint32_t ec_x = 0, ec_y = 0, en_x = 0, en_y = 0;
  int eb = e0;
  if (e0 + lane < e1) {
    const uint2 t = p.entries[e0 + lane];
    ec_x = t.x;
    ec_y = t.y;
  }
  if (e0 + 64 + lane < e1) {
    const uint2 t = p.entries[e0 + 64 + lane];
    en_x = t.x;
    en_y = t.y;
  }

  auto issue = [&](uint32_t ex, lds_char* ks) {
    const bool extra = (ex >> 31) != 0;
    const int64_t nsrc = extra ? p.n_x : p.n_k;
    int64_t k0 = (int64_t)(ex & 0x7fffffffu) * kBN;
    if (k0 >= nsrc) k0 = 0;  // never produced by the plan; keeps every DMA in bounds
    const uint32_t krs = extra ? krs1 : krs0, vrs = extra ? vrs1 : vrs0;
    const char* kb = (extra ? kb1 : kb0) + k0 * krs;
    const char* vb = (extra ? vb1 : vb0) + k0 * vrs;
    lds_char* vs = ks + TILE;
    if (k0 + kBN <= nsrc) {
      const uint32_t lk = dma_lr * krs, lv = dma_lr * vrs;
#pragma unroll
      for (int ii = 0; ii < NIW; ++ii) {
        const uint32_t row0 = (uint32_t)(RPI * (wave * NIW + ii));
        const uint32_t c16 = c16_of(ii);
        const int off = (wave * NIW + ii) * 1024;
        dma16(kb + row0 * krs + (lk + c16), ks + off);
        dma16(vb + row0 * vrs + (lv + c16), vs + off);
      }
    } else {
      // last block of a source: rows past its end re-read the last row (masked later)
      const uint32_t lim = (uint32_t)(nsrc - 1 - k0);
#pragma unroll
      for (int ii = 0; ii < NIW; ++ii) {
        uint32_t r = (uint32_t)(RPI * (wave * NIW + ii)) + dma_lr;
        r = r < lim ? r : lim;
        const uint32_t c16 = c16_of(ii);
        const int off = (wave * NIW + ii) * 1024;
        dma16(kb + (r * krs + c16), ks + off);
        dma16(vb + (r * vrs + c16), vs + off);
      }
    }
  };

  // Q fragments (B operand of S^T = K Q^T): row i32 of this wave, d = 16c + 8h .. +7.
  v8 qf[ND];
  const int64_t my_row = r0 + 32 * wave + i32;
  {
    const int64_t qr = my_row < nrows ? my_row : (int64_t)nrows - 1;
    const char* qp = qbase + qr * qrs + 16 * h;
#pragma unroll
    for (int c = 0; c < ND; ++c) qf[c] = *reinterpret_cast<const v8*>(qp + 32 * c);
  }

  // LDS read offsets (relative to a stage).
  const int sw_k = swz<D>(i32 & 15);
  int koff[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) koff[c] = i32 * RB + ((((2 * c + h) ^ sw_k)) << 4);
  const int g16 = lane & 15;
  const int rowA = 4 * h + (g16 >> 2);            // + 16*s (+8 for the second read)
  const int sw_a = swz<D>(rowA), sw_b = swz<D>(rowA + 8);
  const int dgrp = (lane >> 4) & 1;
  int voffA[NT], voffB[NT];
#pragma unroll
  for (int dt = 0; dt < NT; ++dt) {
    const int chunk = 4 * dt + 2 * dgrp + ((lane & 3) >> 1);
    const int inb = (lane & 1) * 8;
    voffA[dt] = rowA * RB + ((chunk ^ sw_a) << 4) + inb;
    voffB[dt] = (rowA + 8) * RB + ((chunk ^ sw_b) << 4) + inb;
  }

  floatx16 oacc[NT];
#pragma unroll
  for (int dt = 0; dt < NT; ++dt) oacc[dt] = floatx16{0};
  float m_run = -1e30f;                  // running max of s*scale*log2(e)
  float l4[4] = {0.f, 0.f, 0.f, 0.f};    // this lane's share of the row sum, 4 partials
  const float cs = p.scale_log2;
  const int my_tile_row = 32 * wave + i32;

  // One block.  STG (0/1) is the LDS stage of this block, a compile-time
  // constant so every LDS address is a register plus an immediate.
  uint32_t nx = 0, ny = 0;   // entry of the next block (uniform)
  auto body = [&](auto stg_c, int e) {
    constexpr int STG = decltype(stg_c)::value;
    const uint32_t cx = nx, cy = ny;
    wait_vm0();          // this block has landed (the only DMA in flight)
    __syncthreads();     // ... for every wave; the other stage is free again
    if (e + 1 < e1) {
      if (e + 1 - eb == 64) {
        eb += 64;
        ec_x = en_x;
        ec_y = en_y;
        en_x = en_y = 0;
        if (eb + 64 + lane < e1) {
          const uint2 t = p.entries[eb + 64 + lane];
          en_x = t.x;
          en_y = t.y;
        }
      }
      nx = __builtin_amdgcn_readlane(ec_x, e + 1 - eb);
      ny = __builtin_amdgcn_readlane(ec_y, e + 1 - eb);
      issue(nx, smem + (1 - STG) * STAGE);
    }
    const lds_char* ks = smem + STG * STAGE;
    const lds_char* vs = ks + TILE;

    // S^T for keys [0, 32) and [32, 64) of the block.
    floatx16 s0 = floatx16{0}, s1 = floatx16{0};
#pragma unroll
    for (int c = 0; c < ND; ++c) {
      const v8 a0 = *reinterpret_cast<const __attribute__((address_space(3))) v8*>(ks + koff[c]);
      const v8 a1 = *reinterpret_cast<const __attribute__((address_space(3))) v8*>(ks + koff[c] + 32 * RB);
      s0 = O::mfma(a0, qf[c], s0);
      s1 = O::mfma(a1, qf[c], s1);
    }

    // Masks (bit r of `keep`: register r%16 of key half r/16).
    const uint32_t kind = cy & 3u;
    if (kind != kKindNone) {
      const uint32_t keep = block_keep_bits(p, cx, cy, my_tile_row, my_row, nrows, h);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] = ((keep >> r) & 1u) ? s0[r] : -INFINITY;
        s1[r] = ((keep >> (r + 16)) & 1u) ? s1[r] : -INFINITY;
      }
    }

    v8 pb[4];
    if constexpr (D >= 192) {
      // D >= 192: one wave per SIMD issues both the MFMAs and the softmax, so
      // every softmax instruction counts.  The lazy-rescale test reads the
      // block's row sum instead of its row max: P = 2^(s*cs - m) is formed
      // against the running max of the earlier blocks; the running max has
      // to move only if some P exceeds 2^8, and then this lane's share of the
      // row sum (ls) exceeds 2^8 too.  The rare path (and the first block,
      // whose running max is -1e30) takes the true row max and recomputes P.
      auto exps = [&](float nm, float& ls) __attribute__((always_inline)) {
        ls = 0.f;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const floatx16& src = (st < 2) ? s0 : s1;
          const int base = 8 * (st & 1);
          v2 pk[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float a = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * j], cs, nm));
            const float b = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * j + 1], cs, nm));
            pk[j] = O::pack(a, b);
            ls = O::dot2(pk[j], ls);
          }
          pb[st] = v8{pk[0][0], pk[0][1], pk[1][0], pk[1][1], pk[2][0], pk[2][1], pk[3][0], pk[3][1]};
        }
      };
      float ls;
      exps(-m_run, ls);
      if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(ls <= 256.0f)) != 0, 0)) {
        float t8m[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t8m[i] = fmaxf(fmaxf(s0[2 * i], s0[2 * i + 1]), fmaxf(s1[2 * i], s1[2 * i + 1]));
        float mx = fmaxf(fmaxf(fmaxf(t8m[0], t8m[1]), fmaxf(t8m[2], t8m[3])),
                         fmaxf(fmaxf(t8m[4], t8m[5]), fmaxf(t8m[6], t8m[7])));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx * cs);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
        for (int i = 0; i < 4; ++i) l4[i] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_run = m_new;
        exps(-m_run, ls);
      }
      l4[0] += ls;
    } else {
      // Block row max as a tree (both key halves, then the partner lane).
      float t8m[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t8m[i] = fmaxf(fmaxf(s0[2 * i], s0[2 * i + 1]), fmaxf(s1[2 * i], s1[2 * i + 1]));
      float mx = fmaxf(fmaxf(fmaxf(t8m[0], t8m[1]), fmaxf(t8m[2], t8m[3])),
                       fmaxf(fmaxf(t8m[4], t8m[5]), fmaxf(t8m[6], t8m[7])));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mxs = mx * cs;
      if (__builtin_amdgcn_ballot_w64(mxs > m_run + 8.0f)) {
        const float m_new = fmaxf(m_run, mxs);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
        for (int i = 0; i < 4; ++i) l4[i] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_run = m_new;
      }

      // P = 2^(s*cs - m), packed to the MFMA B operand of each 16-key step.
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const floatx16& src = (st < 2) ? s0 : s1;
        const int base = 8 * (st & 1);
        v2 pk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * j], cs, -m_run));
          const float b = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * j + 1], cs, -m_run));
          pk[j] = O::pack(a, b);
          l4[j] = O::dot2(pk[j], l4[j]);
        }
        pb[st] = v8{pk[0][0], pk[0][1], pk[1][0], pk[1][1], pk[2][0], pk[2][1], pk[3][0], pk[3][1]};
      }

    }

    // O^T += V^T P^T.
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int dt = 0; dt < NT; ++dt) {
        const shortx4 ta = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) shortx4*)(vs + voffA[dt] + 16 * st * RB));
        const shortx4 tb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) shortx4*)(vs + voffB[dt] + 16 * st * RB));
        const shortx8 t8 = shortx8{ta[0], ta[1], ta[2], ta[3], tb[0], tb[1], tb[2], tb[3]};
        oacc[dt] = O::mfma(__builtin_bit_cast(v8, t8), pb[st], oacc[dt]);
      }
    }
  };

  if (e0 < e1) {
    nx = __builtin_amdgcn_readlane(ec_x, 0);
    ny = __builtin_amdgcn_readlane(ec_y, 0);
    issue(nx, smem);
  }
  for (int e = e0; e < e1; e += 2) {
    body(std::integral_constant<int, 0>{}, e);
    if (e + 1 < e1) body(std::integral_constant<int, 1>{}, e + 1);
  }

  // Epilogue: combine the row sum of both halves, normalise, store.
  const float l_run = (l4[0] + l4[1]) + (l4[2] + l4[3]);
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (my_row < nrows && partial) {
    store_text_partial<NT>(obase + my_row * ors, lse + 2 * my_row, h, oacc, m_run, l_tot);
  } else if (my_row < nrows) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    char* op = obase + my_row * ors;
#pragma unroll
    for (int dt = 0; dt < NT; ++dt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = 32 * dt + 8 * rq + 4 * h;
        uint2 pk;
        pk.x = (uint32_t)O::bits(oacc[dt][4 * rq] * inv) | ((uint32_t)O::bits(oacc[dt][4 * rq + 1] * inv) << 16);
        pk.y = (uint32_t)O::bits(oacc[dt][4 * rq + 2] * inv) | ((uint32_t)O::bits(oacc[dt][4 * rq + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(op + 2 * d0) = pk;
      }
    }
    if (lse && h == 0) {
      lse[my_row] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * 0.69314718055994530942f : -INFINITY;
    }
  }
}

// ───────────── ping-pong kernel: 8 waves, 256 query rows per tile ─────────────
//
// Waves w and w + 4 of a 512-thread workgroup run on the same SIMD.  Group 0
// (waves 0-3) and group 1 (waves 4-7) hold 32 query rows per wave and walk
// the same key blocks one phase apart, separated by workgroup barriers:
//
//   phase        0       1       2       3       4   ...
//   group 0    M(0)    S(0)    M(1)    S(1)    M(2)
//   group 1     -      M(0)    S(0)    M(1)    S(1)
//
// M(j): S^T of block j and O += P V of block j - 1 (MFMA fed from LDS);
// S(j): mask, row max, exp and row sums of block j (VALU).  At every phase
// each SIMD runs one wave's MFMAs under the other wave's softmax.  K/V blocks
// rotate through a 4-stage LDS ring: block b is read from phase 2b (S^T,
// group 0) to phase 2b + 3 (P V, group 1), and group 0 DMAs block j + 2 from
// its MFMA phase 2j, about three phases before its first use.
// The four K tiles sit at [0, 4 TILE) and the four V tiles above them, and
// the phase loop is unrolled over 8 phases so every stage is a compile-time
// constant: each LDS read is a VGPR plus an immediate.  M phases are
// branch-free: the V tile of stage 3 starts zeroed and P starts at 0, so the
// P V of block -1 in M(0) adds zero, and the S^T of block n computed in M(n)
// is never used.

constexpr int kPPWaves = 8;
constexpr int kPPThreads = 64 * kPPWaves;
constexpr int kPPBM = 32 * kPPWaves;
constexpr int kStream12BM = 384;  // query rows per tile of the 12-wave single-stream kernel (D = 64)
constexpr int kPPStages = 4;

// Workgroup barrier that nothing crosses: the memory clobber orders LDS and
// global accesses, the scheduling barriers keep arithmetic (the exps of a
// softmax phase) from drifting into the next phase.
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left at their maxima.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// v_permlane32_swap on a copy of x: afterwards {a, b} hold x of lanes 0-31
// and x of lanes 32-63 (one in each), so max(a, b) / a + b combine lanes l
// and l ^ 32.  Written as asm with both registers in/out: the two-result
// builtin of this toolchain loses its second result.  The s_nops cover the
// VALU-write -> permlane-read hazard and the reads of its results.
__device__ __forceinline__ void swap_halves(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// IEEE maximum (v_maximum3_f32 when chained): unlike fmaxf it needs no
// canonicalisation of MFMA results first.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max_halves(float x) {
  float a = x, b = x;
  swap_halves(a, b);
  return vmax(a, b);
}
// Materialise x here: keeps the compiler from sinking the computation of a
// phase's results across the barrier into the phase that consumes them.
template <typename T>
__device__ __forceinline__ void pin(T& x) {
  asm volatile("" : "+v"(x));
}
__device__ __forceinline__ float sum_halves(float x) {
  float a = x, b = x;
  swap_halves(a, b);
  return a + b;
}

template <int D, typename E>
__global__ __launch_bounds__(kPPThreads, 1) void attn_fwd_pp_kernel(AttnParams p) {
  using O = Ops<E>;
  using v8 = typename O::v8;
  using v2 = typename O::v2;
  constexpr int RB = (D == 96 ? 128 : D) * 2;  // bytes per K/V row in LDS (D = 96: the D = 128 pitch)
  constexpr int NCH = RB / 16;            // 16-byte chunks per LDS row
  constexpr int NCV = D / 8;              // of which hold data
  constexpr int TILE = kBN * RB;          // bytes of one K or V block
  constexpr int NI = TILE / 1024;         // 1 KiB DMA instructions per block
  constexpr int NIW = NI / 4;             // per group-1 wave
  constexpr int ND = D / 16;              // MFMA k-steps of S
  constexpr int NT = D / 32;              // 32-wide d tiles of O
  constexpr int RPI = 1024 / RB;          // block rows per DMA instruction
  static_assert(NI % 4 == 0, "tile must split evenly over the DMA waves");

  __shared__ __attribute__((aligned(1024))) char smem_raw[2 * kPPStages * TILE];
  lds_char* smem = (lds_char*)smem_raw;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;      // 0: MFMA on even phases, 1: on odd phases
  const int dw = wave & 3;        // DMA slot of a group-1 wave
  const int h = lane >> 5;
  const int i32 = lane & 31;

  const WorkItem it = map_work(p);
  const int tile = it.tile, head = it.head, batch = it.batch;
  const bool text = it.text;
  const int hk = head / p.group;

  const char* qbase;
  char* obase;
  int64_t qrs, ors;
  int nrows;
  int64_t r0;
  float* lse;
  if (!text) {
    qbase = p.q + 2 * (batch * p.q_str[0] + head * p.q_str[2]);
    obase = p.o + 2 * (batch * p.o_str[0] + head * p.o_str[2]);
    qrs = 2 * p.q_str[1];
    ors = 2 * p.o_str[1];
    nrows = p.n_q;
    r0 = (int64_t)tile * kPPBM;
    lse = p.lse ? p.lse + ((int64_t)batch * p.H + head) * p.n_q : nullptr;
  } else {
    qbase = p.qt + 2 * (batch * p.qt_str[0] + head * p.qt_str[2]);
    obase = p.ot + 2 * (batch * p.ot_str[0] + head * p.ot_str[2]);
    qrs = 2 * p.qt_str[1];
    ors = 2 * p.ot_str[1];
    nrows = p.n_tq;
    r0 = (int64_t)(tile - p.n_vt) * kPPBM;
    lse = p.lse_t ? p.lse_t + ((int64_t)batch * p.H + head) * p.n_tq : nullptr;
    if (p.text_chunks > 1) text_partial_dst<D>(p, it, obase, ors, lse);
  }
  const bool partial = text && p.text_chunks > 1;
  int e0, e1;
  item_entries(p, it, e0, e1);
  const int n = e1 - e0;

  const char* kb0 = p.k + 2 * (batch * p.k_str[0] + hk * p.k_str[2]);
  const char* vb0 = p.v + 2 * (batch * p.v_str[0] + hk * p.v_str[2]);
  const char* kb1 = p.n_x ? p.kx + 2 * (batch * p.kx_str[0] + hk * p.kx_str[2]) : kb0;
  const char* vb1 = p.n_x ? p.vx + 2 * (batch * p.vx_str[0] + hk * p.vx_str[2]) : vb0;
  const uint32_t krs0 = (uint32_t)(2 * p.k_str[1]), vrs0 = (uint32_t)(2 * p.v_str[1]);
  const uint32_t krs1 = (uint32_t)(2 * p.kx_str[1]), vrs1 = (uint32_t)(2 * p.vx_str[1]);

  // DMA geometry of a group-0 wave: instruction ii fills LDS KiB 4*ii + dw
  // of a tile, i.e. block rows (4*ii + dw)*RPI + lane/NCH at physical chunk
  // lane%NCH.  The swizzle of those rows depends on row & 15 = (dw*RPI +
  // lane/NCH) & 15 only, so a lane's byte offset within the block is the
  // same for every instruction of the wave and the instruction adds the
  // uniform 4*ii*RPI rows as the buffer soffset.
  const uint32_t dma_row = (uint32_t)(dw * RPI + lane / NCH);  // row of instruction 0
  const uint32_t dma_c16 = (uint32_t)(((lane % NCH) ^ swz<D>((int)(dma_row & 15))) * 16);
  // D = 96: a lane whose chunk lies past the row's data copies from offset
  // 0x7FFF0000 plus the soffset: past the buffer resource's range for a
  // source below that size (zeros, no memory access), else bytes of the
  // source.  Either way no LDS read touches those chunks.  Row strides are
  // below 16 MiB, so with the soffset of at most 60 rows the sum stays below
  // 2^32.
  auto lane_off = [&](uint32_t row_stride) __attribute__((always_inline)) {
    if constexpr (NCV < NCH) {
      if (dma_c16 >= (uint32_t)(16 * NCV)) return 0x7FFF0000u;
    }
    return __umul24(dma_row, row_stride) + dma_c16;
  };

  // Plan entries, 64 per VGPR batch (lane i holds entry eb + i) with the
  // following batch prefetched; a uniform entry is read with v_readlane.
  uint32_t ec_x = 0, ec_y = 0, en_x = 0, en_y = 0;
  int eb = e0;
  if (e0 + lane < e1) {
    const uint2 t = p.entries[e0 + lane];
    ec_x = t.x;
    ec_y = t.y;
  }
  if (e0 + 64 + lane < e1) {
    const uint2 t = p.entries[e0 + 64 + lane];
    en_x = t.x;
    en_y = t.y;
  }
  // entry e, eb <= e < eb + 128
  auto entry = [&](int e, uint32_t& x, uint32_t& y) __attribute__((always_inline)) {
    const int d = e - eb;
    if (d < 64) {
      x = __builtin_amdgcn_readlane(ec_x, d);
      y = __builtin_amdgcn_readlane(ec_y, d);
    } else {
      x = __builtin_amdgcn_readlane(en_x, d - 64);
      y = __builtin_amdgcn_readlane(en_y, d - 64);
    }
  };
  // slide the batches once no entry below e is needed any more
  auto advance = [&](int e) __attribute__((always_inline)) {
    if (e - eb >= 64) {
      eb += 64;
      ec_x = en_x;
      ec_y = en_y;
      en_x = en_y = 0;
      if (eb + 64 + lane < e1) {
        const uint2 t = p.entries[eb + 64 + lane];
        en_x = t.x;
        en_y = t.y;
      }
    }
  };

  // DMA of one block as 2*NIW single instructions that the MFMA phase
  // interleaves with its MFMAs: instruction 2*ii (+1) copies 1 KiB of K (V)
  // through a buffer resource that starts at the block's first row and ends
  // after its last row inside the source, so the rows of a source's short
  // last block past its end land as zeros (they are masked by the plan).
  const uint32_t dofk0 = lane_off(krs0);
  const uint32_t dofv0 = lane_off(vrs0);
  struct BlockSrc {
    u32x4 kr, vr;          // buffer resources of the block's K and V rows
    uint32_t krs, vrs;     // row strides (bytes)
    uint32_t dk, dv;       // per-lane offsets
  };
  auto prep = [&](uint32_t ex) __attribute__((always_inline)) {
    const bool extra = (ex >> 31) != 0;
    const int64_t nsrc = extra ? p.n_x : p.n_k;
    int64_t k0 = (int64_t)(ex & 0x7fffffffu) * kBN;
    if (k0 >= nsrc) k0 = 0;  // never produced by the plan; keeps every DMA in bounds
    BlockSrc src;
    src.krs = extra ? krs1 : krs0;
    src.vrs = extra ? vrs1 : vrs0;
    const uint64_t kb = (uint64_t)((extra ? kb1 : kb0) + k0 * src.krs);
    const uint64_t vb = (uint64_t)((extra ? vb1 : vb0) + k0 * src.vrs);
    const int64_t rows = nsrc - k0 < kBN ? nsrc - k0 : kBN;
    // resource words: base [47:0] (stride 0), num_records in bytes, raw 32-bit data format
    src.kr = u32x4{(uint32_t)kb, (uint32_t)(kb >> 32) & 0xFFFFu, (uint32_t)(rows * src.krs), 0x00020000u};
    src.vr = u32x4{(uint32_t)vb, (uint32_t)(vb >> 32) & 0xFFFFu, (uint32_t)(rows * src.vrs), 0x00020000u};
    src.dk = extra ? lane_off(krs1) : dofk0;
    src.dv = extra ? lane_off(vrs1) : dofv0;
    return src;
  };
  auto dma_one = [&](const BlockSrc& src, int bst, int k) __attribute__((always_inline)) {
    const int ii = k >> 1;
    const uint32_t r = (uint32_t)(4 * ii * RPI);
    if (k & 1) dma16_buf(src.vr, src.dv, r * src.vrs, smem + (kPPStages + bst) * TILE + (4 * ii + dw) * 1024);
    else dma16_buf(src.kr, src.dk, r * src.krs, smem + bst * TILE + (4 * ii + dw) * 1024);
  };

  // Q fragments (B operand of S^T = K Q^T): row i32 of this wave, d = 16c + 8h .. +7.
  v8 qf[ND];
  const int64_t my_row = r0 + 32 * wave + i32;
  {
    const int64_t qr = my_row < nrows ? my_row : (int64_t)nrows - 1;
    const char* qp = qbase + qr * qrs + 16 * h;
#pragma unroll
    for (int c = 0; c < ND; ++c) qf[c] = *reinterpret_cast<const v8*>(qp + 32 * c);
    // Q lands here, once: re-defining the fragments through asm leaves no
    // load the compiler would wait for inside the loop, where the hardware
    // counter also counts the K/V copies in flight.
    wait_vm<0>();
#pragma unroll
    for (int c = 0; c < ND; ++c) pin(qf[c]);
  }

  // LDS read offsets (relative to a stage).
  const int sw_k = swz<D>(i32 & 15);
  int koff[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) koff[c] = i32 * RB + ((((2 * c + h) ^ sw_k)) << 4);
  const int g16 = lane & 15;
  const int rowA = 4 * h + (g16 >> 2);            // + 16*s (+8 for the second read)
  const int sw_a = swz<D>(rowA), sw_b = swz<D>(rowA + 8);
  const int dgrp = (lane >> 4) & 1;
  int voffA[NT], voffB[NT];
#pragma unroll
  for (int dt = 0; dt < NT; ++dt) {
    const int chunk = 4 * dt + 2 * dgrp + ((lane & 3) >> 1);
    const int inb = (lane & 1) * 8;
    voffA[dt] = kPPStages * TILE + rowA * RB + ((chunk ^ sw_a) << 4) + inb;
    voffB[dt] = kPPStages * TILE + (rowA + 8) * RB + ((chunk ^ sw_b) << 4) + inb;
  }

  floatx16 oacc[NT];
#pragma unroll
  for (int dt = 0; dt < NT; ++dt) oacc[dt] = floatx16{0};
  floatx16 s0 = floatx16{0}, s1 = floatx16{0};
  v8 pb[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) pb[st] = v8{};
  float m_run = -1e30f;                  // running max of s*scale*log2(e)
  float l4[4] = {0.f, 0.f, 0.f, 0.f};    // this lane's share of the row sum, 4 partials
  const float cs = p.scale_log2;
  const int my_tile_row = 32 * wave + i32;

  // M(j) with K of block j in stage STG and V of block j - 1 in stage STG - 1:
  // S^T (2*ND MFMAs) then O^T += V^T P^T (4*NT MFMAs) as one stream whose LDS
  // operands are read LA MFMAs ahead (3 measured best for D = 128 under its
  // scheduler, 4 for D = 64).
  constexpr int LA = D == 128 ? 3 : 4;
  constexpr int NQK = 2 * ND, NM = NQK + 4 * NT;
  auto mphase = [&](auto stg_c, auto&& after_mfma) __attribute__((always_inline)) {
    constexpr int STG = decltype(stg_c)::value;
    constexpr int VSTG = (STG + kPPStages - 1) & (kPPStages - 1);
    v8 opa[NM];
    s0 = floatx16{0};
    s1 = floatx16{0};
#pragma unroll
    for (int i = -LA; i < NM; ++i) {
      const int li = i + LA;
      if (li < NM) {
        if (li < NQK) {
          opa[li] = *reinterpret_cast<const __attribute__((address_space(3))) v8*>(
              smem + koff[li >> 1] + (li & 1) * 32 * RB + STG * TILE);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        } else {
          const int k = li - NQK, st = k / NT, dt = k % NT;
          const shortx4 ta = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) shortx4*)(smem + voffA[dt] + VSTG * TILE + 16 * st * RB));
          const shortx4 tb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) shortx4*)(smem + voffB[dt] + VSTG * TILE + 16 * st * RB));
          opa[li] = __builtin_bit_cast(v8, shortx8{ta[0], ta[1], ta[2], ta[3], tb[0], tb[1], tb[2], tb[3]});
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
      }
      if (i >= 0) {
        if (i < NQK) {
          if (i & 1) s1 = O::mfma(opa[i], qf[i >> 1], s1);
          else s0 = O::mfma(opa[i], qf[i >> 1], s0);
        } else {
          const int k = i - NQK;
          oacc[k % NT] = O::mfma(opa[i], pb[k / NT], oacc[k % NT]);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        after_mfma(i);
      }
    }
    pin(s0);
    pin(s1);
#pragma unroll
    for (int dt = 0; dt < NT; ++dt) pin(oacc[dt]);
  };

  // S(j): masks, row max, lazy rescale, P = 2^(s*cs - m) packed for the
  // next M phase, row sums.
  auto sphase = [&](int j) __attribute__((always_inline)) {
    advance(e0 + j);
    uint32_t cx, cy;
    entry(e0 + j, cx, cy);
    // Masks (bit r of `keep`: register r%16 of key half r/16).
    const uint32_t kind = cy & 3u;
    if (kind != kKindNone) {
      const uint32_t keep = block_keep_bits(p, cx, cy, my_tile_row, my_row, nrows, h);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] = ((keep >> r) & 1u) ? s0[r] : -INFINITY;
        s1[r] = ((keep >> (r + 16)) & 1u) ? s1[r] : -INFINITY;
      }
    }

    if constexpr (D == 64 || D == 96) {
      // D = 64 and 96: the rescale test reads this block's row sum instead of
      // its row max (3.6% and 1% faster there; at D = 128 it disturbs the
      // register allocation and runs slower).  P = 2^(s*cs - m) is formed against the
      // running max of the earlier blocks, this lane's share summed in ls.
      // The running max has to move only if some P exceeds 2^8, and then ls
      // exceeds 2^8 too: the rare path (and the first block, whose running
      // max is -1e30) takes the block's true row max and recomputes P.
      float ls = 0.f;
      {
        const float nm = -m_run;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const floatx16& src = (st < 2) ? s0 : s1;
          const int base = 8 * (st & 1);
          v2 pk[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float a = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * jj], cs, nm));
            const float b = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * jj + 1], cs, nm));
            pk[jj] = O::pack(a, b);
            ls = O::dot2(pk[jj], ls);
          }
          pb[st] = v8{pk[0][0], pk[0][1], pk[1][0], pk[1][1], pk[2][0], pk[2][1], pk[3][0], pk[3][1]};
        }
      }
      if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(ls <= 256.0f)) != 0, 0)) {
        float mc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float m = vmax(s0[4 * c], s0[4 * c + 1]);
          m = vmax(m, s0[4 * c + 2]);
          m = vmax(m, s0[4 * c + 3]);
          m = vmax(m, s1[4 * c]);
          m = vmax(m, s1[4 * c + 1]);
          m = vmax(m, s1[4 * c + 2]);
          mc[c] = vmax(m, s1[4 * c + 3]);
        }
        const float mx = max_halves(vmax(vmax(mc[0], mc[1]), vmax(mc[2], mc[3])));
        const float m_new = vmax(m_run, mx * cs);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
        for (int i = 0; i < 4; ++i) l4[i] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_run = m_new;
        ls = 0.f;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const floatx16& src = (st < 2) ? s0 : s1;
          const int base = 8 * (st & 1);
          v2 pk[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float a = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * jj], cs, -m_run));
            const float b = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * jj + 1], cs, -m_run));
            pk[jj] = O::pack(a, b);
            ls = O::dot2(pk[jj], ls);
          }
          pb[st] = v8{pk[0][0], pk[0][1], pk[1][0], pk[1][1], pk[2][0], pk[2][1], pk[3][0], pk[3][1]};
        }
      }
      l4[0] += ls;
    } else {
      // block row max: four independent chains of v_maximum3, then the partner lane
      float mc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float m = vmax(s0[4 * c], s0[4 * c + 1]);
        m = vmax(m, s0[4 * c + 2]);
        m = vmax(m, s0[4 * c + 3]);
        m = vmax(m, s1[4 * c]);
        m = vmax(m, s1[4 * c + 1]);
        m = vmax(m, s1[4 * c + 2]);
        mc[c] = vmax(m, s1[4 * c + 3]);
      }
      const float mx = max_halves(vmax(vmax(mc[0], mc[1]), vmax(mc[2], mc[3])));
      const float mxs = mx * cs;
      if (__builtin_amdgcn_ballot_w64(mxs > m_run + 8.0f)) {
        const float m_new = vmax(m_run, mxs);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
        for (int i = 0; i < 4; ++i) l4[i] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_run = m_new;
      }

#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const floatx16& src = (st < 2) ? s0 : s1;
        const int base = 8 * (st & 1);
        v2 pk[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float a = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * jj], cs, -m_run));
          const float b = __builtin_amdgcn_exp2f(__builtin_fmaf(src[base + 2 * jj + 1], cs, -m_run));
          pk[jj] = O::pack(a, b);
          l4[jj] = O::dot2(pk[jj], l4[jj]);
        }
        pb[st] = v8{pk[0][0], pk[0][1], pk[1][0], pk[1][1], pk[2][0], pk[2][1], pk[3][0], pk[3][1]};
      }
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) pin(pb[st]);
#pragma unroll
    for (int i = 0; i < 4; ++i) pin(l4[i]);
    pin(m_run);
#pragma unroll
    for (int dt = 0; dt < NT; ++dt) pin(oacc[dt]);
  };

  // V tile of stage 3 = 0: read by the P V of block -1 in M(0) (with P = 0).
  {
    constexpr int NZ = TILE / (16 * kPPThreads);
#pragma unroll
    for (int z = 0; z < NZ; ++z)
      *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(
          smem + (2 * kPPStages - 1) * TILE + (z * kPPThreads + (int)threadIdx.x) * 16) = u32x4{0, 0, 0, 0};
  }
  __syncthreads();

  // Block b of the plan, or a stand-in past the end: row 0 of a key source,
  // DMA'd into a stage that is never read again (keeps every MFMA phase the
  // same instruction stream and the DMA count per phase constant).
  const uint32_t stand_in = p.n_k > 0 ? 0u : 0x80000000u;
  auto block_src = [&](int b) __attribute__((always_inline)) {
    uint32_t x = stand_in, y;
    if (b < n) entry(e0 + b, x, y);
    return prep(x);
  };

  // Prologue: group 0 starts blocks 0 and 1; block 0 lands before phase 0.
  if (grp == 0) {
    const BlockSrc s0b = block_src(0);
#pragma unroll
    for (int k = 0; k < 2 * NIW; ++k) dma_one(s0b, 0, k);
    const BlockSrc s1b = block_src(1);
#pragma unroll
    for (int k = 0; k < 2 * NIW; ++k) dma_one(s1b, 1, k);
    wait_vm<2 * NIW>();
  }
  wg_barrier();

  // Group 0 runs phases 0 .. 2n: M(j) on phase 2j, S(j) on phase 2j + 1;
  // group 1 runs them one phase later.  Both pass 2n + 1 barriers.  Group 0
  // owns the DMA and spreads it over its MFMA phases (one instruction after
  // every fourth MFMA): M(j) copies block j + 2, whose stage last held block
  // j - 2 (read for the last time by group 1's M(j - 1) on phase 2j - 1), and
  // S(j) ends with block j + 1 landed for M(j + 1) (only block j + 2 may
  // still be in flight).  Blocks are processed 4 at a time so the stage of
  // every block is a compile-time constant.
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  constexpr int CI = NM / (2 * NIW);      // MFMAs per copy instruction (4; 3 for D = 96)
  static_assert(CI >= 1 && 2 * NIW * CI <= NM, "copies must fit the MFMA phase");
  if (grp == 0) {
    auto mdma = [&](auto stg_c, int b) __attribute__((always_inline)) {
      constexpr int BST = (decltype(stg_c)::value + 2) & (kPPStages - 1);
      const BlockSrc src = block_src(b);
      mphase(stg_c, [&](int i) __attribute__((always_inline)) {
        if (i % CI == CI - 1 && i / CI < 2 * NIW) {  // after the last MFMA of each group of CI
          dma_one(src, BST, i / CI);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
      });
    };
    for (int j0 = 0;; j0 += 4) {
      mdma(I0{}, j0 + 2);
      wg_barrier();
      if (j0 >= n) break;
      sphase(j0);
      wait_vm<2 * NIW>();
      wg_barrier();
      mdma(I1{}, j0 + 3);
      wg_barrier();
      if (j0 + 1 >= n) break;
      sphase(j0 + 1);
      wait_vm<2 * NIW>();
      wg_barrier();
      mdma(I2{}, j0 + 4);
      wg_barrier();
      if (j0 + 2 >= n) break;
      sphase(j0 + 2);
      wait_vm<2 * NIW>();
      wg_barrier();
      mdma(I3{}, j0 + 5);
      wg_barrier();
      if (j0 + 3 >= n) break;
      sphase(j0 + 3);
      wait_vm<2 * NIW>();
      wg_barrier();
    }
    wait_vm<0>();  // stand-in copies still in flight land before the workgroup ends
  } else {
    auto none = [](int) {};
    wg_barrier();
    for (int j0 = 0;; j0 += 4) {
      mphase(I0{}, none);
      if (j0 >= n) break;
      wg_barrier();
      sphase(j0);
      wg_barrier();
      mphase(I1{}, none);
      if (j0 + 1 >= n) break;
      wg_barrier();
      sphase(j0 + 1);
      wg_barrier();
      mphase(I2{}, none);
      if (j0 + 2 >= n) break;
      wg_barrier();
      sphase(j0 + 2);
      wg_barrier();
      mphase(I3{}, none);
      if (j0 + 3 >= n) break;
      wg_barrier();
      sphase(j0 + 3);
      wg_barrier();
    }
  }

  // Epilogue: combine the row sum of both halves, normalise, store.
  const float l_run = (l4[0] + l4[1]) + (l4[2] + l4[3]);
  const float l_tot = sum_halves(l_run);
  if (my_row < nrows && partial) {
    store_text_partial<NT>(obase + my_row * ors, lse + 2 * my_row, h, oacc, m_run, l_tot);
  } else if (my_row < nrows) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    char* op = obase + my_row * ors;
#pragma unroll
    for (int dt = 0; dt < NT; ++dt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = 32 * dt + 8 * rq + 4 * h;
        uint2 pk;
        pk.x = (uint32_t)O::bits(oacc[dt][4 * rq] * inv) | ((uint32_t)O::bits(oacc[dt][4 * rq + 1] * inv) << 16);
        pk.y = (uint32_t)O::bits(oacc[dt][4 * rq + 2] * inv) | ((uint32_t)O::bits(oacc[dt][4 * rq + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(op + 2 * d0) = pk;
      }
    }
    if (lse && h == 0) {
      lse[my_row] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * 0.69314718055994530942f : -INFINITY;
    }
  }
}

template <int D, typename E>
int launch(const AttnParams& prm, int block_q, hipStream_t stream) {
  if constexpr (D == 96) {
    (void)block_q;
    hipLaunchKernelGGL((attn_fwd_pp_kernel<D, E>), dim3(prm.total_work), dim3(kPPThreads), 0, stream, prm);
    return launch_status("lvsa_attn_fwd");
  }
  if constexpr (D == 64 || D == 128) {
    if (block_q == kPPBM) {
      hipLaunchKernelGGL((attn_fwd_pp_kernel<D, E>), dim3(prm.total_work), dim3(kPPThreads), 0, stream, prm);
      return launch_status("lvsa_attn_fwd");
    }
  }
  if constexpr (D != 96) {
    hipLaunchKernelGGL((attn_fwd_kernel<D, E>), dim3(prm.total_work), dim3(kThreads), 0, stream, prm);
  }
  return launch_status("lvsa_attn_fwd");
}

}  // namespace
}  // namespace lvsa

