"""Frame-run and token-interval helpers of the one-GPU path (the single-GPU part of src/onereel/parallel/comm.py:
`merge` :69-77, `clip` :80-81, `frame_tokens` :84-85, `runs` :115-123), and the rank token ranges of a split layer
(`query_cost` :17-22, Algorithm 1 `balanced` :25-40, `partition` :43-66).

On the device these runs are implicit: the layout kernel walks each scope's key frames and writes their token rows.
The host helpers serve callers of the reference module. A rank range from `partition` is what the layout takes as
its query range (q_lo, q_hi) to run one rank's share of the layer; the exchange of the K/V rows a rank reads from
other ranks (halo exchange, Ulysses all-to-all) is not part of the one-GPU path.
"""
from __future__ import annotations

from itertools import groupby

# the reference's fitted per-query cost u = C_LIN + C_ATT * EFF_SCENE * L' (ms per video token and forward, L' keys
# per query; HunyuanVideo-1.5 720p on one H200, comm.py:11-15): only the ratio C_ATT / C_LIN moves the boundaries
C_LIN, C_ATT, EFF_SCENE = 0.02581842, 6.753627e-07, 1.0


def merge(iv) -> list:
    """the union of half-open intervals as sorted, disjoint intervals; intervals that touch are joined and empty
    ones dropped"""
    out = []
    for lo, hi in sorted((a, b) for a, b in iv if a < b):
        if out and lo <= out[-1][1]:
            out[-1] = (out[-1][0], max(out[-1][1], hi))
        else:
            out.append((lo, hi))
    return out


def clip(iv, a: int, b: int) -> list:
    """each interval intersected with [a, b); intervals outside it dropped"""
    return [(max(lo, a), min(hi, b)) for lo, hi in iv if hi > a and lo < b]


def runs(frames) -> list:
    """maximal stretches of frames that rise by one, in list order: [3, 4, 5, 1, 2] -> [(3, 6), (1, 3)]"""
    out = []
    for _, grp in groupby(enumerate(frames), key=lambda p: p[1] - p[0]):
        fs = [f for _, f in grp]
        out.append((fs[0], fs[-1] + 1))
    return out


def frame_tokens(frames, T: int) -> list:
    """the token rows of a frame list (frame-major, T tokens per frame) as intervals, one per run of frames"""
    return [(lo * T, hi * T) for lo, hi in runs(frames)]


def query_cost(layout, T: int, text=None, extra_keys: int = 0, c_lin: float = C_LIN, c_att: float = C_ATT) -> list:
    """per scene, the modelled cost of one of its video queries: c_lin + c_att * EFF_SCENE * (its key frames' tokens
    + its sentence's tokens + extra_keys) (comm.py:17-22)"""
    text = text or [0] * layout.n_scenes
    return [c_lin + c_att * EFF_SCENE * (len(layout.key_frames(j)) * T + text[j] + extra_keys)
            for j in range(layout.n_scenes)]


def balanced(sizes, cost, n: int) -> list:
    """Algorithm 1 (comm.py:25-40): scenes in order, sizes[j] queries of cost cost[j] each; boundary p (0 < p < n)
    goes to the query at which the running work reaches p / n of the total, rounded to the nearest query of the scene
    it falls in, then clamped so that every rank keeps at least one query. A scene is cut only where a boundary falls
    inside it. -> per rank (first query, end query)."""
    L = sum(sizes)
    if L < n:
        raise ValueError(f'{L} queries for {n} ranks')
    work = [m * c for m, c in zip(sizes, cost)]
    prefix = [0.0]
    for w in work:
        prefix.append(prefix[-1] + w)
    share = prefix[-1] / n
    bounds, j, first = [0], 0, 0          # scene j starts at query `first`, after prefix[j] of the work
    for p in range(1, n):
        goal = p * share
        # the first scene whose end reaches the goal (a relative slack of 1e-12 keeps a goal that lands on a scene
        # end in that scene rather than at the start of the next)
        while j < len(sizes) - 1 and prefix[j + 1] < goal - 1e-12 * prefix[-1]:
            first += sizes[j]
            j += 1
        at = first + int(round((goal - prefix[j]) / cost[j]))
        bounds.append(min(max(at, bounds[-1] + 1), L - (n - p)))
    bounds.append(L)
    return list(zip(bounds[:-1], bounds[1:]))


def partition(layout, n: int, T: int, mode: str, text=None, extra_keys: int = 0, granularity: str = 'balanced') -> list:
    """rank video-token ranges (frame-major, T tokens per frame; comm.py:43-66). mode 'ulysses' (or n = 1): equal
    ranges, the tokens dividing evenly. mode 'scene' (K/V gathering): granularity 'balanced' is Algorithm 1 over the
    scenes' modelled query costs, 'tokens' equal ranges, 'scenes' the balanced boundaries moved to the nearest scene
    start (no scene cut)."""
    S = layout.n_frames * T
    if mode == 'ulysses' or n == 1:
        if S % n:
            raise ValueError(f'{S} video tokens do not split evenly over {n} ranks')
        return [(r * S // n, (r + 1) * S // n) for r in range(n)]
    if mode != 'scene':
        raise ValueError(f"mode must be 'scene' or 'ulysses', got {mode!r}")
    if granularity == 'tokens':
        return [(r * S // n, (r + 1) * S // n) for r in range(n)]
    if granularity not in ('balanced', 'scenes'):
        raise ValueError(f"granularity must be 'balanced', 'tokens' or 'scenes', got {granularity!r}")
    own = balanced([m * T for m in layout.lengths], query_cost(layout, T, text, extra_keys), n)
    if granularity == 'balanced':
        return own
    if layout.n_scenes < n:
        raise ValueError(f'{layout.n_scenes} scenes for {n} ranks')
    starts = [lo * T for lo, _ in layout.ranges]
    bounds = [0]
    for p in range(1, n):
        # scene starts after the previous boundary that leave a scene for each later rank; ties go to the earlier
        ok = [s for i, s in enumerate(starts) if i > 0 and s > bounds[-1] and i <= layout.n_scenes - (n - p)]
        bounds.append(min(ok, key=lambda s: abs(s - own[p][0])))
    bounds.append(S)
    return list(zip(bounds[:-1], bounds[1:]))
