"""CPU restatement of LVSA's frame-granularity mask — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module; the product never does.

Every function restates the reference implementation in
``lvsa/sparse_attention.py`` (LVSA v1.2.0) and cites the lines it follows.
The restatement is written independently (different control flow where the
reference is procedural) but must agree bit-for-bit; tests pin it against
golden vectors produced from the reference itself, against the reference's
own known-answer tests, and against brute-force characterisations.

Conventions: frames are latent frames ``0..T-1``; a token ``t`` of the
(full, world=1) video sequence lives in frame ``t // P``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, Iterable, List, Optional, Sequence, Set, Tuple

# ─────────────────────────────────────────────────────────────────────────────
# Scalar helpers
# ─────────────────────────────────────────────────────────────────────────────


def adaptive_window_bounds(f: int, W: int, T: int) -> Tuple[int, int]:
    """Constant-width window shifted at the sequence edges.

    Follows ``lvsa/sparse_attention.py:40-47``: the nominal window
    ``[f-W, f+W]`` is slid right at the start and left at the end so it keeps
    ``min(2W+1, T)`` frames.
    """
    lo = min(f - W, T - 1 - 2 * W)
    hi = max(f + W, 2 * W)
    return max(0, lo), min(T - 1, hi)


def expanded_window_bounds(
    f: int, W: int, T: int, global_set: Set[int], global_count: int
) -> Tuple[int, int]:
    """Grow the adaptive window until it holds ``min(2W+1, T-|G|)`` non-global frames.

    Follows ``lvsa/sparse_attention.py:50-86``.  Restated as a move sequence:
    the window edges are pushed alternately left, right, left, right, ...
    (a push that would leave ``[0, T-1]`` is skipped); growth stops the moment
    the non-global count reaches the target, or when two consecutive pushes
    are both impossible.
    """
    lo, hi = adaptive_window_bounds(f, W, T)
    need = min(2 * W + 1, T - global_count)
    have = sum(1 for x in range(lo, hi + 1) if x not in global_set)
    go_left = True
    blocked = 0
    while have < need and blocked < 2:
        if go_left and lo > 0:
            lo -= 1
            added = lo
        elif (not go_left) and hi < T - 1:
            hi += 1
            added = hi
        else:
            added = None
        go_left = not go_left
        if added is None:
            blocked += 1
            continue
        blocked = 0
        if added not in global_set:
            have += 1
    return lo, hi


def get_window_bounds(
    f: int, W: int, T: int, expand: bool, global_set: Set[int], global_count: int
) -> Tuple[int, int]:
    """``lvsa/sparse_attention.py:89-104``: W=0 gives the empty range (f, f-1)."""
    if W == 0:
        return f, f - 1
    if expand:
        return expanded_window_bounds(f, W, T, global_set, global_count)
    return adaptive_window_bounds(f, W, T)


def compute_global_indices(
    total_frames: int, n_first_frames: int, key_frame_interval: Optional[int], offset: int = 0
) -> List[int]:
    """Anchor frames ∪ rotated keyframe grid, sorted.

    ``lvsa/sparse_attention.py:198-216``: the first ``n_first`` frames plus
    ``ceil(T/kfi)`` keyframes ``(offset + i*kfi) mod T`` (modular wrap, so the
    count is the same for every offset).
    """
    T = total_frames
    out = set(range(min(n_first_frames, T)))
    kfi = key_frame_interval
    if kfi is not None and kfi > 0:
        n_key = -(-T // kfi)
        out.update((offset + i * kfi) % T for i in range(n_key))
    return sorted(out)


def compute_boundary_guard_frames(
    total_frames: int, local_seq: int, num_patches: int, world: int, window_size: int
) -> List[int]:
    """Frames within ±W of every context-parallel token split.

    ``lvsa/sparse_attention.py:107-129``.
    """
    out: Set[int] = set()
    for r in range(1, world):
        b = (r * local_seq) // num_patches
        lo = max(0, b - window_size)
        hi = min(total_frames, b + window_size + 1)
        out.update(range(lo, hi))
    return sorted(out)


def compute_auto_kfi(
    total_frames: int,
    window_size: int,
    n_first_frames: int,
    reference_frames: int = 21,
    sparsity_scale: float = 1.0,
) -> int:
    """Keyframe interval targeting ``reference_frames * sparsity_scale`` attended frames.

    ``lvsa/sparse_attention.py:132-195``: max of the largest interval whose
    anchor set still reaches the target global count and a closed-form
    fallback ``ceil((T - mandatory) / (ref - mandatory))``.
    """
    T, W, n = total_frames, window_size, n_first_frames
    ref = max(n + 1, int(reference_frames * sparsity_scale))
    if T <= ref:
        return 1
    want_globals = max(n, min(ref, T) - min(2 * W + 1, T))
    strict = 1
    for kfi in range(T, 0, -1):
        size = len(set(range(min(n, T))) | set(range(0, T, kfi)))
        if size >= want_globals:
            strict = kfi
            break
    mandatory = 2 * W + n
    fallback = math.ceil(max(T - mandatory, ref - mandatory) / max(ref - mandatory, 1))
    return max(strict, fallback)


# ─────────────────────────────────────────────────────────────────────────────
# Frame-level mask and its CSR
# ─────────────────────────────────────────────────────────────────────────────


@dataclass
class FrameMask:
    """Everything ``LVSAMetadata.build`` derives from the pattern parameters.

    Field meanings follow ``lvsa/sparse_attention.py:286-333``.
    """

    T: int
    P: int
    local_seq: int
    gts: int
    global_indices: List[int]
    window_bounds: List[Tuple[int, int]]          # per frame 0..T-1
    local_frames: List[Tuple[int, int, int]]
    window_ctx: Dict[int, List[Tuple[int, int]]]
    rows: List[List[int]]                         # per CSR q-block: sorted attended frames
    compact_frames: List[int]
    indptr: List[int]
    indices: List[int]
    MB: int
    global_copies: List[Tuple[int, int]]
    local_copies: List[Tuple[int, int]]
    attended_rows: List[List[int]] = field(default_factory=list)  # _build_attended_indices rows

    @property
    def global_set(self) -> Set[int]:
        return set(self.global_indices)

    @property
    def compact_n(self) -> int:
        return len(self.compact_frames)


def build_frame_mask(
    T: int,
    P: int,
    W: int,
    n_first: int,
    kfi: Optional[int],
    rank: int = 0,
    world: int = 1,
    expand: bool = True,
    offset: int = 0,
    guards: Optional[Sequence[int]] = None,
) -> FrameMask:
    """Restates ``LVSAMetadata.build`` (``lvsa/sparse_attention.py:335-484``)
    together with ``_build_attended_indices`` (``:510-547``) and
    ``_build_flashinfer_csr`` (``:550-635``).

    The CSR has ``MB = ceil(local_seq/P)`` rows, row ``qi`` describing frame
    ``gts//P + qi``; a row holds every global frame plus each non-global
    window frame that has tokens on this rank; column ids are positions in
    the sorted union of all rows (``compact_frames``).
    """
    total = T * P
    if total % world:
        raise AssertionError("T*P must be divisible by world")
    local = total // world
    gts = rank * local
    G = sorted(set(compute_global_indices(T, n_first, kfi, offset)) | set(guards or ()))
    Gs = set(G)
    nG = len(G)

    def bounds(f: int) -> Tuple[int, int]:
        return get_window_bounds(f, W, T, expand, Gs, nG)

    def local_span(fr: int) -> Tuple[int, int]:
        return max(fr * P, gts), min((fr + 1) * P, gts + local)

    first = gts // P
    last = (gts + local - 1) // P
    local_frames = []
    for fr in range(first, last + 1):
        s, e = local_span(fr)
        local_frames.append((fr, s - gts, e - gts))

    window_ctx: Dict[int, List[Tuple[int, int]]] = {}
    for fr, _, _ in local_frames:
        lo, hi = bounds(fr)
        parts = []
        for wf in range(lo, hi + 1):
            if wf in Gs:
                continue
            s, e = local_span(wf)
            if s < e:
                parts.append((s - gts, e - gts))
        window_ctx[fr] = parts

    window_bounds = [bounds(fr) for fr in range(T)]

    attended_rows = []
    for fr in range(first, last + 1):
        lo, hi = bounds(fr)
        attended_rows.append(sorted(Gs | set(range(lo, hi + 1))))

    MB = -(-local // P)
    rows: List[List[int]] = []
    for qi in range(MB):
        fr = first + qi
        lo, hi = bounds(fr)
        row = set(G)
        for wf in range(lo, hi + 1):
            if wf not in Gs:
                s, e = local_span(wf)
                if s < e:
                    row.add(wf)
        rows.append(sorted(row))
    compact = sorted(set().union(*rows)) if rows else []
    pos = {fr: i for i, fr in enumerate(compact)}
    indptr = [0]
    indices: List[int] = []
    for row in rows:
        indices.extend(pos[fr] for fr in row)
        indptr.append(len(indices))
    gpos = {fr: i for i, fr in enumerate(G)}
    gcop, lcop = [], []
    for ci, fr in enumerate(compact):
        if fr in Gs:
            gcop.append((gpos[fr] * P, ci * P))
        else:
            lcop.append((fr * P - gts, ci * P))
    return FrameMask(
        T=T, P=P, local_seq=local, gts=gts, global_indices=G,
        window_bounds=window_bounds, local_frames=local_frames, window_ctx=window_ctx,
        rows=rows, compact_frames=compact, indptr=indptr, indices=indices, MB=MB,
        global_copies=gcop, local_copies=lcop, attended_rows=attended_rows,
    )


def frame_relation(mask: FrameMask) -> List[Set[int]]:
    """Per q-frame (world=1) set of attended key frames: the CSR rows as sets."""
    return [set(r) for r in mask.rows]


def window_only_relation(mask: FrameMask) -> List[Set[int]]:
    """Per q-frame set of key frames reached through ``window_ctx`` only
    (non-global window frames).  This is what ``lvsa_sdpa`` reads from ``key``
    besides the pre-gathered ``k_global`` (``lvsa/sparse_attention.py:677-687``).
    """
    P, out = mask.P, []
    for fr, _, _ in mask.local_frames:
        s = set()
        for a, b in mask.window_ctx[fr]:
            s.update(range((a + mask.gts) // P, (b - 1 + mask.gts) // P + 1))
        out.append(s)
    return out


# ─────────────────────────────────────────────────────────────────────────────
# Token-level refinement
# ─────────────────────────────────────────────────────────────────────────────


def block_csr(
    relation: Sequence[Set[int]], P: int, n_q: int, n_k: int, bq: int, bk: int
) -> Tuple[List[int], List[int]]:
    """Canonical-grid block CSR of a frame relation.

    Query block ``i`` covers tokens ``[i*bq, min((i+1)*bq, n_q))``, key block
    ``j`` covers ``[j*bk, min((j+1)*bk, n_k))``; the pair is active iff some
    query token's frame attends some key token's frame.  Brute force over
    frame pairs (the relation is frame-granular).
    """
    nqb, nkb = -(-n_q // bq), -(-n_k // bk)
    indptr, cols = [0], []
    for i in range(nqb):
        qf = range((i * bq) // P, (min((i + 1) * bq, n_q) - 1) // P + 1)
        keys = set()
        for f in qf:
            keys |= relation[f]
        for j in range(nkb):
            kf0, kf1 = (j * bk) // P, (min((j + 1) * bk, n_k) - 1) // P
            if any(g in keys for g in range(kf0, kf1 + 1)):
                cols.append(j)
        indptr.append(len(cols))
    return indptr, cols


def token_mask(relation: Sequence[Set[int]], P: int, n_q: int, n_k: int):
    """Dense boolean ``[n_q, n_k]`` token mask of a frame relation (small shapes only)."""
    import numpy as np

    T_q = -(-n_q // P)
    T_k = -(-n_k // P)
    fm = np.zeros((T_q, T_k), dtype=bool)
    for f in range(T_q):
        for g in relation[f]:
            if g < T_k:
                fm[f, g] = True
    qf = np.arange(n_q) // P
    kf = np.arange(n_k) // P
    return fm[qf][:, kf]


def block_flops(relation: Sequence[Set[int]], P: int, n_v: int, bq: int, bk: int,
                H: int, D: int, n_t: int = 0, batch: int = 1) -> Tuple[int, int]:
    """Algorithmic FLOPs of one attention call.

    Returns ``(block, token_exact)``:
    ``4·B·H·D·[Σ_active |qblk|·|kblk| + N_v·N_t + N_t·(N_v+N_t)]`` on the
    canonical grid, and the same with the mask's token count in place of the
    block area.
    """
    nqb, nkb = -(-n_v // bq), -(-n_v // bk)
    indptr, cols = block_csr(relation, P, n_v, n_v, bq, bk)
    area = 0
    for i in range(nqb):
        qn = min((i + 1) * bq, n_v) - i * bq
        for j in cols[indptr[i]:indptr[i + 1]]:
            area += qn * (min((j + 1) * bk, n_v) - j * bk)
    T = n_v // P
    exact = sum(P * P * len(relation[f]) for f in range(T))
    dense_text = n_v * n_t + n_t * (n_v + n_t)
    k = 4 * batch * H * D
    return k * (area + dense_text), k * (exact + dense_text)
