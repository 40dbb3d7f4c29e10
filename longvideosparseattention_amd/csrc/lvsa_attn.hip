// Block-sparse flash-attention forward for LVSA on gfx950 (MI355X): the C ABI
// entry point (lvsa_attn_fwd), its argument checks and the dispatch by head
// size.  The kernels are in lvsa_attn_kernels.h, instantiated per head size
// in lvsa_attn_d64.hip, lvsa_attn_d96.hip, lvsa_attn_d128.hip,
// lvsa_attn_d192.hip and lvsa_attn_d256.hip.
#include "lvsa_attn_kernels.h"

namespace {

bool aligned16(const void* ptr, const int64_t* str, int n) {
  if (((uintptr_t)ptr) % 16) return false;
  for (int i = 0; i < n; ++i)
    if ((str[i] * 2) % 16) return false;
  return true;
}

}  // namespace

using namespace lvsa;

extern "C" int lvsa_attn_fwd(const lvsa_attn_args* a, hipStream_t stream) {
  clear_error();
  LVSA_REQUIRE(a != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: null args");
  LVSA_REQUIRE(a->D == 64 || a->D == 96 || a->D == 128 || a->D == 192 || a->D == 256, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: head_dim %d not supported (64, 96, 128, 192, 256)", a->D);
  LVSA_REQUIRE(a->D < 192 || a->block_q == kBM, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: head_dim %d runs 128-row tiles (block_q %d)", a->D, a->block_q);
  LVSA_REQUIRE(a->D != 96 || a->block_q == kPPBM, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: head_dim 96 runs 256-row tiles (block_q %d)", a->block_q);
  LVSA_REQUIRE(a->dtype == LVSA_BF16 || a->dtype == LVSA_FP16, LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd: dtype %d",
               a->dtype);
  LVSA_REQUIRE(a->B >= 1 && a->H >= 1 && a->Hkv >= 1 && a->H % a->Hkv == 0, LVSA_ERR_INVALID_ARG,
               "lvsa_attn_fwd: B=%d H=%d Hkv=%d (H must be a multiple of Hkv)", a->B, a->H, a->Hkv);
  LVSA_REQUIRE(a->n_q >= 0 && a->n_k >= 0 && a->n_x >= 0 && a->n_tq >= 0, LVSA_ERR_INVALID_ARG,
               "lvsa_attn_fwd: negative length");
  LVSA_REQUIRE(a->tile_indptr && a->entries, LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd: missing plan");
  LVSA_REQUIRE(a->block_q == kBM || a->block_q == kPPBM, LVSA_ERR_UNSUPPORTED,
               "lvsa_attn_fwd: block_q %d (the kernels tile 128 or 256 query rows)", a->block_q);
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
  if (a->n_q) ok = ok && aligned16(a->q, a->q_str, 3) && aligned16(a->o, a->o_str, 3);
  if (a->n_tq) ok = ok && aligned16(a->qt, a->qt_str, 3) && aligned16(a->ot, a->ot_str, 3);
  if (a->n_k) ok = ok && aligned16(a->k, a->k_str, 3) && aligned16(a->v, a->v_str, 3);
  if (a->n_x) ok = ok && aligned16(a->kx, a->kx_str, 3) && aligned16(a->vx, a->vx_str, 3);
  LVSA_REQUIRE(ok, LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd: tensors must be 16-byte aligned with 16-byte row strides");
  // per-lane DMA offsets within a 64-row key block are 32-bit
  auto fits = [&](int64_t row_elems) { return row_elems >= 0 && row_elems * 2 * (kBN - 1) + 2LL * a->D <= 0xFFFFFFFFLL; };
  LVSA_REQUIRE(fits(a->k_str[1]) && fits(a->v_str[1]) && (a->n_x == 0 || (fits(a->kx_str[1]) && fits(a->vx_str[1]))),
               LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd: key/value row stride too large");
  // the 256-row kernel forms per-lane row offsets with 24-bit multiplies
  auto fits24 = [&](int64_t row_elems) { return row_elems * 2 < (1LL << 24); };
  LVSA_REQUIRE(a->block_q != kPPBM || (fits24(a->k_str[1]) && fits24(a->v_str[1]) &&
                                       (a->n_x == 0 || (fits24(a->kx_str[1]) && fits24(a->vx_str[1])))),
               LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd: key/value row stride of 16 MiB or more (block_q 256)");
  const int64_t work = (int64_t)a->n_tiles * a->H * a->B;
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
  const int bq = a->block_q;
  if (a->D == 256) return launch_d256(p, bq, a->dtype == LVSA_BF16, stream);
  if (a->D == 128) return launch_d128(p, bq, a->dtype == LVSA_BF16, stream);
  if (a->D == 96) return launch_d96(p, bq, a->dtype == LVSA_BF16, stream);
  if (a->D == 192) return launch_d192(p, bq, a->dtype == LVSA_BF16, stream);
  return launch_d64(p, bq, a->dtype == LVSA_BF16, stream);
}
