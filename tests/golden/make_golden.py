"""Write golden vectors of LVSA's frame-mask functions from the reference.

Run in the build container (the reference is never shipped anywhere):

    python tests/golden/make_golden.py --reference /root/reference

It imports the reference package ``lvsa.sparse_attention`` from the given
checkout and records, as JSON data only, the outputs of the functions whose
exact behaviour no test of the reference pins down:

* ``expanded_window_bounds`` / ``get_window_bounds`` (alternating tie-break),
* ``compute_global_indices`` (modular keyframe rotation),
* ``compute_auto_kfi``,
* ``LVSAMetadata.build`` — window bounds, local frames, window context,
  attended-index table and the FlashInfer CSR with its compact numbering and
  copy lists,

over the BASELINE configurations (all keyframe offsets) and a seeded random
grid of small geometries (including context-parallel ranks).  The output file
``lvsa_mask_golden.json.gz`` is consumed by ``tests/test_oracle_golden.py`` (CPU)
and ``tests/test_gpu_mask.py`` (GPU).
"""

from __future__ import annotations

import argparse
import gzip
import json
import random
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent

BASELINE = [
    # name, T, P, W, n_first, kfi, offsets
    ("cpu", 9, 256, 1, 1, 4, [3]),
    ("wan4x", 84, 1560, 2, 1, 8, list(range(8))),
    ("wan6x_w1", 121, 1560, 1, 1, 8, list(range(8))),
    ("wan6x_w2", 121, 1560, 2, 1, 8, list(range(8))),
    ("wan6x_w4", 121, 1560, 4, 1, 8, list(range(8))),
    ("cog", 13, 1350, 1, 1, 4, list(range(4))),
    ("hv", 49, 1590, 2, 1, 8, list(range(8))),
]


def metadata_record(sa, T, P, W, n, kfi, rank, world, expand, offset, guards, full=True):
    m = sa.LVSAMetadata.build(
        total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=n,
        key_frame_interval=kfi, rank=rank, world=world, expand_window=expand,
        keyframe_offset=offset, boundary_guards=guards,
    )
    rec = {
        "args": {"T": T, "P": P, "W": W, "n_first": n, "kfi": kfi, "rank": rank, "world": world,
                 "expand": expand, "offset": offset, "guards": guards},
        "global_indices": list(m.global_indices),
        "window_bounds": m.window_bounds.tolist(),
        "fi_indptr": m.fi_indptr.tolist(),
        "fi_indices": m.fi_indices.tolist(),
        "fi_M": m.fi_M, "fi_N": m.fi_N, "fi_MB": m.fi_MB, "fi_compact_n": m.fi_compact_n,
        "local_seq": m.local_seq, "global_token_start": m.global_token_start,
    }
    if full:
        rec.update({
            "local_frames": [list(x) for x in m.local_frames],
            "window_ctx": {str(k): [list(p) for p in v] for k, v in m.window_ctx.items()},
            "attended_indices": m.attended_indices.tolist(),
            "attended_C": m.attended_C,
            "fi_global_copies": [list(x) for x in m.fi_global_copies],
            "fi_local_copies": [list(x) for x in m.fi_local_copies],
            "global_frame_mask": m.global_frame_mask.tolist(),
        })
    return rec


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--reference", required=True, help="path of the reference checkout")
    ap.add_argument("--out", default=str(HERE / "lvsa_mask_golden.json.gz"))
    ap.add_argument("--seed", type=int, default=20261201)
    args = ap.parse_args(argv)
    sys.path.insert(0, args.reference)
    import lvsa.sparse_attention as sa  # noqa: E402  (reference, build container only)

    out = {"source": "lvsa.sparse_attention (LVSA v1.2.0)", "seed": args.seed,
           "baseline": [], "random": [], "windows": [], "auto_kfi": []}

    for name, T, P, W, n, kfi, offsets in BASELINE:
        for off in offsets:
            rec = metadata_record(sa, T, P, W, n, kfi, 0, 1, True, off, None, full=False)
            rec["name"] = name
            out["baseline"].append(rec)

    rng = random.Random(args.seed)
    n_rand = 0
    while n_rand < 360:
        T = rng.randint(1, 40)
        P = rng.randint(1, 9)
        W = rng.choice([0, 1, 1, 2, 2, 3, 4, 6])
        n = rng.randint(0, 3)
        kfi = rng.choice([None, 0, 1, 2, 3, 4, 5, 7, 8, T, T + 3])
        offset = rng.randint(0, max(0, (kfi or 1) - 1) + 2)
        expand = rng.random() < 0.8
        world = rng.choice([1, 1, 1, 2, 3, 4])
        if (T * P) % world:
            continue
        rank = rng.randrange(world)
        guards = None
        if world > 1 and rng.random() < 0.7:
            guards = sa.compute_boundary_guard_frames(T, T * P // world, P, world, W)
        if n == 0 and (kfi is None or kfi == 0) and not guards and W == 0:
            continue  # reference rows would be empty (no attended frame at all)
        try:
            rec = metadata_record(sa, T, P, W, n, kfi, rank, world, expand, offset, guards)
        except (AssertionError, ValueError, KeyError, RuntimeError) as exc:  # record failures too
            rec = {"args": {"T": T, "P": P, "W": W, "n_first": n, "kfi": kfi, "rank": rank, "world": world,
                            "expand": expand, "offset": offset, "guards": guards},
                   "error": type(exc).__name__}
        out["random"].append(rec)
        n_rand += 1

    # Window bounds with arbitrary (not keyframe-shaped) global sets.
    for _ in range(600):
        T = rng.randint(1, 60)
        W = rng.randint(0, 7)
        G = sorted(rng.sample(range(T), rng.randint(0, T)))
        f = rng.randrange(T)
        expand = rng.random() < 0.85
        lo, hi = sa.get_window_bounds(f, W, T, expand, set(G), len(G))
        out["windows"].append({"f": f, "W": W, "T": T, "G": G, "expand": expand, "bounds": [lo, hi]})

    for _ in range(300):
        T = rng.randint(1, 200)
        W = rng.randint(0, 12)
        n = rng.randint(1, 8)
        ref = rng.choice([21, 33, 13, 6])
        scale = rng.choice([0.5, 0.8, 1.0, 1.0, 1.5, 2.0])
        out["auto_kfi"].append({"T": T, "W": W, "n_first": n, "ref": ref, "scale": scale,
                                "kfi": sa.compute_auto_kfi(T, W, n, reference_frames=ref, sparsity_scale=scale)})

    with gzip.open(args.out, "wt", compresslevel=9) as fh:
        json.dump(out, fh, separators=(",", ":"))
    print(f"wrote {args.out}: {len(out['baseline'])} baseline, {len(out['random'])} random, "
          f"{len(out['windows'])} window, {len(out['auto_kfi'])} auto-kfi records")
    return 0


if __name__ == "__main__":
    sys.exit(main())
