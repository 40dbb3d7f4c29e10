/*
 * lvsa_amd.h — C ABI of the MI355X (gfx950) LVSA sparse-attention library.
 *
 * The library implements the hot path of LVSA (Long-Video Sparse Attention,
 * JiusiServe/LongVideoSparseAttention v1.2.0) as HIP kernels:
 *
 *   1. lvsa_mask_build  — the frame-granularity mask builder (anchor frames,
 *      rotated keyframe grid, adaptive/expanded sliding window) emitting the
 *      frame-level block CSR on device, bit-exact with the reference's
 *      FlashInfer CSR.
 *   2. lvsa_plan_build  — the token-level refinement of a frame relation into
 *      block-sparse row-pointer / column-index lists on the canonical
 *      (block_q x block_k) grid, with per-block mask descriptors.
 *   3. lvsa_attn_fwd    — block-sparse flash-attention forward (bf16/fp16 MFMA)
 *      over those lists, with dense "extra" key rows (text tokens or a
 *      pre-gathered global K/V) and dense text query rows.
 *
 * Conventions
 *   - Plain pointers and sizes only.  Device pointers are HIP device memory
 *     owned by the caller; nothing is allocated or freed inside.
 *   - Every entry point only enqueues work on the given stream (no host
 *     synchronisation, no device allocation), so calls are graph-capturable.
 *   - Return value: LVSA_OK (0) or a negative lvsa_status; the message of the
 *     last failure on the calling thread is available from lvsa_last_error().
 *   - Tensors are [B, S, H, D] with arbitrary element strides for B, S and H
 *     and a contiguous last dimension (stride 1).
 */
#ifndef LVSA_AMD_H
#define LVSA_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LVSA_API __attribute__((visibility("default")))

#define LVSA_AMD_VERSION "0.1.0"
#define LVSA_MAX_FRAMES 4096          /* T limit of the mask builder          */
#define LVSA_BITMAP_WORDS (LVSA_MAX_FRAMES / 32)

typedef enum lvsa_status {
  LVSA_OK = 0,
  LVSA_ERR_INVALID_ARG = -1,   /* bad size, null pointer, inconsistent geometry */
  LVSA_ERR_UNSUPPORTED = -2,   /* head_dim / dtype / stride not supported         */
  LVSA_ERR_CAPACITY = -3,      /* caller buffer smaller than the stated bound     */
  LVSA_ERR_HIP = -4            /* a HIP runtime call failed (launch error)        */
} lvsa_status;

/* LVSA_FP32: fp32 in and out, fp32 products and accumulation (the reference
 * computes in the caller's dtype, lvsa/sparse_attention.py:670, 689-704);
 * 128-row tiles, text tiles unsplit.                                        */
typedef enum lvsa_dtype { LVSA_BF16 = 0, LVSA_FP16 = 1, LVSA_FP32 = 2 } lvsa_dtype;

/* ───────────────────────── frame mask builder ─────────────────────────── */

/* Pattern parameters of LVSAMetadata.build
 * (reference: lvsa/sparse_attention.py:339-353; the caller passes the keyframe
 * offset, i.e. step % kfi, as in lvsa/lvsa_processor.py:317-331).           */
typedef struct lvsa_mask_params {
  int32_t T;            /* total latent frames (1..LVSA_MAX_FRAMES)              */
  int32_t P;            /* tokens per latent frame                              */
  int32_t window;       /* W >= 0; 0 = globals-only                             */
  int32_t n_first;      /* anchor frames 0..n_first-1                           */
  int32_t kfi;          /* key-frame interval; <= 0 means "None"                */
  int32_t offset;       /* keyframe-grid rotation                               */
  int32_t expand;       /* 1 = expanded window (reference default), 0 = adaptive */
  int32_t rank;         /* context-parallel position; (0, 1) on one GPU         */
  int32_t world;
  uint32_t guard_bits[LVSA_BITMAP_WORDS]; /* boundary-guard frames, bit f = frame f */
  /* Device re-tune (set_window_size / set_sparsity_scale,
   * lvsa/lvsa_processor.py:288-315, 333-360): with auto_kfi = 1 the builder
   * derives kfi from (T, window, n_first, reference_frames, sparsity_scale)
   * as lvsa_auto_kfi does and uses offset = step % kfi; the kfi and offset
   * fields are then ignored.  info[7] reports the kfi used either way.      */
  int32_t auto_kfi;
  int32_t reference_frames;  /* reference default 21                         */
  double sparsity_scale;     /* reference default 1.0                        */
  int64_t step;              /* denoising step index (>= 0)                  */
} lvsa_mask_params;

/* Output sizes of lvsa_mask_build (all int32 unless noted):
 *   n_rows        MB = ceil(local_seq/P): CSR rows (q frames of this rank)
 *   n_local       frames holding local tokens (MB or MB+1)
 *   words         bitmap words per row = ceil(T/32)
 *   max_nnz       capacity bound for frame_indices (n_rows * T)             */
typedef struct lvsa_mask_sizes {
  int32_t n_rows, n_local, words, max_nnz;
  int64_t local_seq, global_token_start;
} lvsa_mask_sizes;

/* Replaces the sizing part of LVSAMetadata.build (lvsa/sparse_attention.py:355-364). */
LVSA_API int lvsa_mask_sizes_query(const lvsa_mask_params* p, lvsa_mask_sizes* out);

/* Device outputs of the mask builder (caller-allocated):
 *   frame_indptr   [n_rows+1]        CSR row pointers       == fi_indptr
 *   frame_indices  [max_nnz]         compact column ids     == fi_indices
 *   compact_frames [T]               compact id -> frame (first compact_n valid)
 *   global_frames  [T]               sorted global frames (first n_global valid)
 *   window_bounds  [T*2]             (lo, hi) per frame     == window_bounds
 *   rel_full       [n_local*words]   uint32 bitmap: row = local frame,
 *                                    bit g = frame g attended (globals + window)
 *   rel_window     [n_local*words]   uint32 bitmap of window_ctx frames only
 *   info           [8]               nnz, compact_n, n_global, n_rows,
 *                                    n_local, first_frame, max_row_nnz,
 *                                    kfi used (0 = none)                      */
typedef struct lvsa_mask_out {
  int32_t* frame_indptr;
  int32_t* frame_indices;
  int32_t* compact_frames;
  int32_t* global_frames;
  int32_t* window_bounds;
  uint32_t* rel_full;
  uint32_t* rel_window;
  int32_t* info;
} lvsa_mask_out;

/* Replaces compute_global_indices + get_window_bounds + _build_flashinfer_csr
 * (lvsa/sparse_attention.py:89-104, 198-216, 550-635) as called from
 * LVSAMetadata.build (:335-484).  One work-group; enqueue only.              */
LVSA_API int lvsa_mask_build(const lvsa_mask_params* p, const lvsa_mask_out* out, hipStream_t stream);

/* compute_auto_kfi (lvsa/sparse_attention.py:132-195) on the device:
 * *kfi_out (device int32) = the keyframe interval that gives about
 * int(reference_frames * sparsity_scale) attended frames per query frame for
 * T frames, window W and n_first anchors.  Used by the processor's re-tune
 * (lvsa/lvsa_processor.py:303-309, 348-354).  One work-group; enqueue only. */
LVSA_API int lvsa_auto_kfi(int32_t T, int32_t window, int32_t n_first, int32_t reference_frames,
                           double sparsity_scale, int32_t* kfi_out, hipStream_t stream);

/* ─────────────────────── block plan (token refinement) ──────────────────── */

/* A frame relation refined to the canonical token-block grid.
 *   q row r of source "q" lives in q-frame (q_tok0 + r) / R,
 *   key row c of source 0 lives in key-frame (k_tok0 + c) / C;
 *   relation row (qframe - q_frame0) of `rel` lists the attended key frames.
 * Source 1 ("extra", n_x rows) is attended by every video query row; text
 * query rows (n_tq) attend every row of both sources.
 * Replaces the FlashInfer plan over the reference CSR
 * (lvsa/lvsa_processor.py:768-830, lvsa-vllm-omni/lvsa_vllm_omni/flashinfer_runner.py:71-94)
 * and the per-frame context assembly of lvsa_sdpa (lvsa/sparse_attention.py:674-687). */
typedef struct lvsa_plan_params {
  int32_t n_q, n_k, n_x, n_tq;
  int32_t R, C;
  int64_t q_tok0, k_tok0;
  int32_t q_frame0;
  int32_t rel_rows, words;
  const uint32_t* rel;      /* device bitmap [rel_rows*words]                     */
  int32_t block_q, block_k; /* query tile rows (128/256/384) x key block (64)     */
} lvsa_plan_params;

typedef struct lvsa_plan_sizes {
  int32_t n_tiles;          /* video tiles + text tiles                           */
  int32_t n_video_tiles;
  int64_t max_entries;      /* capacity bound for the entry list                  */
  int64_t workspace_bytes;  /* scratch for lvsa_plan_build                        */
} lvsa_plan_sizes;

/* Host-side sizing; `max_row_frames` bounds the attended frames per relation row
 * (pass T when unknown).                                                       */
LVSA_API int lvsa_plan_sizes_query(const lvsa_plan_params* p, int32_t max_row_frames, lvsa_plan_sizes* out);

/* Device outputs:
 *   tile_indptr [n_tiles+1] int32; entries [max_entries] 2 x uint32 each:
 *     word0 = (source << 31) | key-block index
 *     word1 = mask descriptor: bits 0-1 kind (0 none, 1 two-part, 2 generic),
 *             bits 2-5 allow bits (qa.lo, qa.hi, qb.lo, qb.hi),
 *             bits 8-15 key split within the block, bits 16-24 row split
 *             (255 when the tile has a single query part).
 *   block_q <= 384, block_k <= 255; lvsa_attn_fwd runs tiles of 128, 256 or
 *   (head size 64, 16-bit, frames of at least 383 query and 64 key rows) 384
 *   query rows (lvsa_attn_args.block_q) over key blocks of 64.               */
LVSA_API int lvsa_plan_build(const lvsa_plan_params* p, int32_t* tile_indptr, uint32_t* entries,
                    int64_t max_entries, void* workspace, int64_t workspace_bytes,
                    hipStream_t stream);

/* Block CSR (row pointers, column ids) -> relation bitmap [n_rows*words]
 * (bit c of row r set iff column c is listed in row r).  Used to plan a
 * block-sparse wrapper from the CSR it was given, as FlashInfer's
 * BlockSparseAttentionWrapper.plan does (lvsa/lvsa_processor.py:805-827;
 * flashinfer_runner.py:79-94).  status[0] = 1 flags out-of-range columns.
 * status needs 4 int32 (the last two are scratch).                          */
LVSA_API int lvsa_csr_to_bitmap(const int32_t* indptr, const int32_t* indices, int32_t n_rows, int32_t n_cols,
                                uint32_t* bitmap, int32_t words, int32_t* status, hipStream_t stream);

/* ─────────────────────────── attention forward ─────────────────────────── */

typedef struct lvsa_attn_args {
  /* tensors: q/o [B, n_q, H, D]; k/v [B, n_k, Hkv, D]; kx/vx [B, n_x, Hkv, D];
   * qt/ot [B, n_tq, H, D].  kx/vx/qt/ot may be null when the count is 0.       */
  const void* q; const void* k; const void* v;
  const void* kx; const void* vx; const void* qt;
  void* o; void* ot;
  float* lse;               /* optional [B, H, n_q] natural-log LSE             */
  float* lse_t;             /* optional [B, H, n_tq]                            */
  int64_t q_str[3], k_str[3], v_str[3], kx_str[3], vx_str[3], qt_str[3], o_str[3], ot_str[3];
  int32_t B, H, Hkv, D;      /* D = 64, 96, 128, 192 or 256                      */
  int32_t n_q, n_k, n_x, n_tq;
  float scale;              /* softmax scale (reference: 1/sqrt(D))             */
  int32_t dtype;            /* lvsa_dtype                                       */
  /* plan (built with block_q = 128, 256 or 384 query rows and block_k = 64;
   * D = 256 and fp32 run 128-row tiles only, D = 96 256-row tiles only,
   * 384-row tiles are for D = 64 in 16 bit; D = 192 in 16 bit runs 128-row
   * tiles, or 256-row ones on the dual-wide map for frames of >= 255 query
   * and >= 64 key rows whose frame source's short last key block lies in one
   * frame, from sources below 2^31 bytes: other 256-row calls at D = 192
   * return LVSA_ERR_UNSUPPORTED) */
  int32_t block_q;
  const int32_t* tile_indptr;
  const uint32_t* entries;
  int32_t n_tiles, n_video_tiles;
  /* relation for generic (kind 2) blocks: row (q_tok0 + r)/R - q_frame0 of
   * rel [rel_rows x words] serves query row r, so every query row must fall
   * inside it (checked)                                                       */
  const uint32_t* rel; int32_t words, R, C, q_frame0;
  int64_t q_tok0, k_tok0;
  int32_t rel_rows;
  /* optional scratch (device memory, lvsa_attn_workspace_query bytes, 16-byte
   * aligned; its contents on entry do not matter).  With it:
   * - each text-query tile's key range is split into chunks that run as
   *   separate work items after the video tiles and are merged by a second
   *   launch (exact log-sum-exp merge, as flashinfer_runner.py:184-197), so
   *   the long text tiles fill the launch's last round instead of
   *   lengthening it;
   * - the single-stream kernel (every 16-bit head size) runs one persistent
   *   work-group per CU (two for head size 64) that takes work items from
   *   eight per-XCD queues (counters in the last 1 KiB, zeroed by the call)
   *   and steals from the other XCDs' queues once its own is empty, so XCDs
   *   that run faster take over items of slower ones;
   * - at head size 64 (two work-groups per CU) each queue's last video
   *   tiles run as two key-range halves each, merged by a third launch as
   *   the text chunks are, when the scratch holds their partials (the size
   *   lvsa_attn_workspace_query returns; a smaller scratch of at least the
   *   text split and the counters runs the tiles whole).
   * Null: one work-group per work item, text tiles whole and first.          */
  void* workspace;
  int64_t workspace_bytes;
} lvsa_attn_args;

/* Replaces lvsa_sdpa's per-frame loop (lvsa/sparse_attention.py:643-706), the
 * FlashInfer block-sparse run + dense text term + LSE merge
 * (lvsa/lvsa_processor.py:832-913; flashinfer_runner.py:96-198) and the dense
 * encoder-query attention (lvsa/lvsa_processor.py:710-735) with one launch.   */
LVSA_API int lvsa_attn_fwd(const lvsa_attn_args* a, hipStream_t stream);

/* Bytes of scratch lvsa_attn_fwd uses for `a`: the text-tile split
 * partials (none without text queries), the video-tile split partials (head
 * size 64, when the call has enough tiles for the work queues; their number
 * follows the current device's compute units) and 1 KiB of work-queue
 * counters; host only, nothing is launched.
 * Replaces the float workspace the FlashInfer wrapper is planned with
 * (flashinfer_runner.py:75-79, lvsa/lvsa_processor.py:798-804: 128 MB).      */
LVSA_API int lvsa_attn_workspace_query(const lvsa_attn_args* a, int64_t* bytes);

/* lvsa_attn_fwd without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  It has no counterpart in the reference.  The
 * scratch (work-queue counters and the text-tile split) comes from a static
 * device array of LVSA_NOALLOC_SCRATCH_BYTES per GPU (a->workspace is
 * ignored), which each GPU the library runs on holds until the process
 * ends; a call whose text split and counters need more returns
 * LVSA_ERR_CAPACITY (the video split runs only when it fits as well).  All calls on one GPU share that array: calls
 * that overlap on one GPU (other streams, other threads) race, so serialise
 * them.  The caller still passes inputs and outputs; nothing else differs
 * from lvsa_attn_fwd.                                                         */
#define LVSA_NOALLOC_SCRATCH_BYTES (64LL << 20)
LVSA_API int lvsa_attn_fwd_noalloc(const lvsa_attn_args* a, hipStream_t stream);

/* Gather K/V rows of whole frames into a packed buffer (dst[b, i*P + t] =
 * src[b, frames[i]*P + t]).  Replaces build_global_kv
 * (lvsa-vllm-omni/lvsa_vllm_omni/global_kv.py:12-42) and the single-GPU copy
 * of DistributedLVSAProcessor._build_global_kv (lvsa/lvsa_processor.py:643-706). */
LVSA_API int lvsa_gather_frames(const void* src, const int64_t src_str[3], void* dst, const int64_t dst_str[3],
                       const int32_t* frames, int32_t n_frames, int32_t P,
                       int32_t B, int32_t H, int32_t D, int32_t elem_bytes, hipStream_t stream);

/* Library identification and error reporting. */
LVSA_API const char* lvsa_version(void);
LVSA_API const char* lvsa_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* LVSA_AMD_H */
