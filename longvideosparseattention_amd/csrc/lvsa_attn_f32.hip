// fp32 attention for fp32 callers (gfx950).
//
// The reference's lvsa_sdpa computes in the caller's dtype
// (lvsa/sparse_attention.py:670, 689-704): an fp32 caller gets fp32 scores,
// softmax and P.V.  This kernel keeps that: Q, K, V and O stay fp32, both
// contractions run on v_mfma_f32_32x32x2_f32 (fp32 products, fp32
// accumulation), and the online softmax is exact (the running max moves with
// every block that raises it).  It walks the same block plan as the 16-bit
// kernels (128-row tiles, 64-key blocks, the same mask descriptors) with the
// same accumulator layout, so masks use block_keep_bits unchanged.
//
// Per wave (32 query rows) and key block:
//   S^T = K Q^T   A = K[key][d] (lane l: key l%32 of a 32-key half, d from
//                 a float4 at 8g + 4(l/32)), B = Q (registers), the four
//                 components of the float4 as four k-steps;
//   O^T += V^T P^T  k-step c of key half kh pairs keys 32kh + 8(c/4) + c%4
//                 and +4 (lane halves), i.e. the keys whose P this lane
//                 already holds in accumulator register c: B = that register,
//                 A = V[key][32dt + l%32] (one LDS dword per lane).
// K and V blocks are staged through padded LDS rows (D + 4 floats) by plain
// vector loads, one barrier pair per block.  fp32 MFMA peak is 157 TFLOP/s;
// this path trades speed for the caller's precision and is not the
// throughput path.
#include "lvsa_attn_kernels.h"

namespace lvsa {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int D>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_f32_kernel(AttnParams p) {
  constexpr int PITCH = D + 4;   // floats per LDS row
  constexpr int NG = D / 8;      // float4 pairs of S's contraction
  constexpr int NT = D / 32;     // 32-wide d tiles of O
  constexpr int C4 = D / 4;      // float4 per K/V row
  __shared__ __attribute__((aligned(16))) float ks[kBN * PITCH];
  __shared__ __attribute__((aligned(16))) float vs[kBN * PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;
  const int i32 = lane & 31;

  const WorkItem it = map_work(p);
  const int tile = it.tile, head = it.head, batch = it.batch;
  const int hk = head / p.group;

  const char* qbase;
  char* obase;
  int64_t qrs, ors;
  int nrows;
  int64_t r0;
  float* lse;
  if (!it.text) {
    qbase = p.q + 4 * (batch * p.q_str[0] + head * p.q_str[2]);
    obase = p.o + 4 * (batch * p.o_str[0] + head * p.o_str[2]);
    qrs = 4 * p.q_str[1];
    ors = 4 * p.o_str[1];
    nrows = p.n_q;
    r0 = (int64_t)tile * kBM;
    lse = p.lse ? p.lse + ((int64_t)batch * p.H + head) * p.n_q : nullptr;
  } else {
    qbase = p.qt + 4 * (batch * p.qt_str[0] + head * p.qt_str[2]);
    obase = p.ot + 4 * (batch * p.ot_str[0] + head * p.ot_str[2]);
    qrs = 4 * p.qt_str[1];
    ors = 4 * p.ot_str[1];
    nrows = p.n_tq;
    r0 = (int64_t)(tile - p.n_vt) * kBM;
    lse = p.lse_t ? p.lse_t + ((int64_t)batch * p.H + head) * p.n_tq : nullptr;
  }
  int e0, e1;
  item_entries(p, it, e0, e1);

  const char* kb0 = p.k + 4 * (batch * p.k_str[0] + hk * p.k_str[2]);
  const char* vb0 = p.v + 4 * (batch * p.v_str[0] + hk * p.v_str[2]);
  const char* kb1 = p.n_x ? p.kx + 4 * (batch * p.kx_str[0] + hk * p.kx_str[2]) : kb0;
  const char* vb1 = p.n_x ? p.vx + 4 * (batch * p.vx_str[0] + hk * p.vx_str[2]) : vb0;

  // Q of row i32: components d = 8g + 4h .. +3 in q[4g ..].
  const int64_t my_row = r0 + 32 * wave + i32;
  float q[D / 2];
  {
    const int64_t qr = my_row < nrows ? my_row : (int64_t)nrows - 1;
    const char* qp = qbase + qr * qrs + 16 * h;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const floatx4 t = *reinterpret_cast<const floatx4*>(qp + 32 * g);
      q[4 * g] = t[0];
      q[4 * g + 1] = t[1];
      q[4 * g + 2] = t[2];
      q[4 * g + 3] = t[3];
    }
  }

  floatx16 oacc[NT];
#pragma unroll
  for (int dt = 0; dt < NT; ++dt) oacc[dt] = floatx16{0};
  float m_run = -1e30f;   // running max of s * scale * log2(e)
  float l_run = 0.f;      // this lane's share of the row sum
  const float cs = p.scale_log2;
  const int my_tile_row = 32 * wave + i32;

  for (int e = e0; e < e1; ++e) {
    const uint2 ent = p.entries[e];
    const uint32_t cx = ent.x, cy = ent.y;
    const bool extra = (cx >> 31) != 0;
    const int64_t nsrc = extra ? p.n_x : p.n_k;
    int64_t k0 = (int64_t)(cx & 0x7fffffffu) * kBN;
    if (k0 >= nsrc) k0 = 0;   // never produced by the plan; keeps every load in bounds
    const char* kb = extra ? kb1 : kb0;
    const char* vb = extra ? vb1 : vb0;
    const int64_t krs = 4 * (extra ? p.kx_str[1] : p.k_str[1]);
    const int64_t vrs = 4 * (extra ? p.vx_str[1] : p.v_str[1]);

    __syncthreads();   // the previous block's LDS reads are done
    for (int idx = tid; idx < kBN * C4; idx += kThreads) {
      const int row = idx / C4, c = idx - row * C4;
      int64_t key = k0 + row;
      key = key < nsrc ? key : nsrc - 1;   // rows past the source end are masked by the descriptor
      *reinterpret_cast<floatx4*>(&ks[row * PITCH + 4 * c]) = *reinterpret_cast<const floatx4*>(kb + key * krs + 16 * c);
      *reinterpret_cast<floatx4*>(&vs[row * PITCH + 4 * c]) = *reinterpret_cast<const floatx4*>(vb + key * vrs + 16 * c);
    }
    __syncthreads();

    floatx16 s0 = floatx16{0}, s1 = floatx16{0};
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const floatx4 a0 = *reinterpret_cast<const floatx4*>(&ks[i32 * PITCH + 8 * g + 4 * h]);
      const floatx4 a1 = *reinterpret_cast<const floatx4*>(&ks[(32 + i32) * PITCH + 8 * g + 4 * h]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], q[4 * g + t], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], q[4 * g + t], s1, 0, 0, 0);
      }
    }

    if ((cy & 3u) != kKindNone) {
      const uint32_t keep = block_keep_bits(p, cx, cy, my_tile_row, my_row, nrows, h);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] = ((keep >> r) & 1u) ? s0[r] : -INFINITY;
        s1[r] = ((keep >> (r + 16)) & 1u) ? s1[r] : -INFINITY;
      }
    }

    // Exact online softmax: the row max over both lanes of the row.
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx * cs);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int dt = 0; dt < NT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], cs, -m_run));
      s1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], cs, -m_run));
      l_run += s0[r] + s1[r];
    }

#pragma unroll
    for (int dt = 0; dt < NT; ++dt) {
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const int key = 8 * (c >> 2) + 4 * h + (c & 3);
        const float a0 = vs[key * PITCH + 32 * dt + i32];
        const float a1 = vs[(32 + key) * PITCH + 32 * dt + i32];
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, s0[c], oacc[dt], 0, 0, 0);
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, s1[c], oacc[dt], 0, 0, 0);
      }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (my_row < nrows) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    char* op = obase + my_row * ors;
#pragma unroll
    for (int dt = 0; dt < NT; ++dt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = 32 * dt + 8 * rq + 4 * h;
        *reinterpret_cast<floatx4*>(op + 4 * d0) =
            floatx4{oacc[dt][4 * rq] * inv, oacc[dt][4 * rq + 1] * inv, oacc[dt][4 * rq + 2] * inv,
                    oacc[dt][4 * rq + 3] * inv};
      }
    }
    if (lse && h == 0) lse[my_row] = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.69314718055994530942f : -INFINITY;
  }
}

}  // namespace

int launch_f32(const AttnParams& prm, int D, hipStream_t stream) {
  const dim3 grid(prm.total_work), block(kThreads);
  switch (D) {
    case 64: hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, grid, block, 0, stream, prm); break;
    case 96: hipLaunchKernelGGL(attn_fwd_f32_kernel<96>, grid, block, 0, stream, prm); break;
    case 128: hipLaunchKernelGGL(attn_fwd_f32_kernel<128>, grid, block, 0, stream, prm); break;
    case 192: hipLaunchKernelGGL(attn_fwd_f32_kernel<192>, grid, block, 0, stream, prm); break;
    default: hipLaunchKernelGGL(attn_fwd_f32_kernel<256>, grid, block, 0, stream, prm); break;
  }
  return launch_status("lvsa_attn_fwd (fp32)");
}

}  // namespace lvsa
