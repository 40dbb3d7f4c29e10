// Host-side check of the work-queue map of the single-stream kernel
// (lvsa_attn_kernels.h: queue_shape, queue_item): over random geometries,
// every video tile is taken exactly once, whole or as its two key-range
// halves, every text item exactly once, and each split tile's halves use the
// partial slot from which attn_video_merge_kernel (lvsa_attn.hip) reads it
// back.  Prints "queue map ok" and exits 0, or names the first failure.
#include "lvsa_attn_kernels.h"

#include <cstdio>
#include <random>
#include <vector>

using namespace lvsa;

int main() {
  std::mt19937 rng(1);
  for (int trial = 0; trial < 20000; ++trial) {
    AttnParams p{};
    p.B = 1 + rng() % 3;
    p.H = 1 + rng() % 48;
    p.n_vt = rng() % 40;
    p.n_tt = rng() % 3;
    p.text_chunks = (p.n_tt && rng() % 2) ? 1 + rng() % 9 : 1;
    p.text_first = p.text_chunks == 1;
    p.vsplit = (rng() % 3 == 0) ? 0 : 1 + rng() % 40;
    p.n_vwork = p.n_vt * p.H * p.B;
    p.n_twork = p.n_tt * p.text_chunks * p.H * p.B;
    std::vector<int> seen_v(p.n_vwork, 0), seen_t(p.n_twork, 0), slot_of(p.n_vwork, -1);
    std::vector<int> slot_halves(kXcds * (p.vsplit > 0 ? p.vsplit : 1), 0);
    long total = 0;
    for (int x = 0; x < kXcds; ++x) {
      const QueueShape q = queue_shape(p, x);
      const int len = queue_items(q);
      total += len;
      for (int j = 0; j < len; ++j) {
        const WorkItem it = queue_item(p, x, j);
        if (it.text) {
          const int t = ((it.batch * p.H + it.head) * p.n_tt + (it.tile - p.n_vt)) * p.text_chunks + it.chunk;
          if (t < 0 || t >= p.n_twork || it.tile < p.n_vt || it.vhalf != -1) {
            printf("trial %d: bad text item (queue %d, slot %d)\n", trial, x, j);
            return 1;
          }
          ++seen_t[t];
          continue;
        }
        const int w = (it.batch * p.H + it.head) * p.n_vt + it.tile;
        if (w < 0 || w >= p.n_vwork || it.tile >= p.n_vt) {
          printf("trial %d: bad video item (queue %d, slot %d)\n", trial, x, j);
          return 1;
        }
        if (it.vhalf < 0) {
          seen_v[w] += 2;
          continue;
        }
        seen_v[w] += 1;
        if (it.vslot < 0 || it.vslot >= kXcds * p.vsplit || (slot_of[w] >= 0 && slot_of[w] != it.vslot)) {
          printf("trial %d: bad split slot %d\n", trial, it.vslot);
          return 1;
        }
        slot_of[w] = it.vslot;
        slot_halves[it.vslot] |= 1 << it.vhalf;
        // the merge kernel's map from the slot back to the tile
        const int mx = it.vslot / p.vsplit, sx = it.vslot % p.vsplit;
        const QueueShape mq = queue_shape(p, mx);
        if (sx >= mq.n_split || mq.v0 + mq.n_video - mq.n_split + sx != w) {
          printf("trial %d: merge map of slot %d misses tile %d\n", trial, it.vslot, w);
          return 1;
        }
      }
    }
    for (int w = 0; w < p.n_vwork; ++w) {
      if (seen_v[w] != 2 || (slot_of[w] >= 0 && slot_halves[slot_of[w]] != 3)) {
        printf("trial %d: video item %d taken %d/2 times\n", trial, w, seen_v[w]);
        return 1;
      }
    }
    for (int t = 0; t < p.n_twork; ++t) {
      if (seen_t[t] != 1) {
        printf("trial %d: text item %d taken %d times\n", trial, t, seen_t[t]);
        return 1;
      }
    }
    long splits = 0;
    for (int x = 0; x < kXcds; ++x) splits += queue_shape(p, x).n_split;
    if (total != p.n_vwork + p.n_twork + splits) {
      printf("trial %d: %ld queue slots for %d + %d items and %ld halves\n", trial, total, p.n_vwork, p.n_twork,
             splits);
      return 1;
    }
  }
  printf("queue map ok\n");
  return 0;
}
