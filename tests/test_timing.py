"""Word-timestamp kernels: DTW (triton_ops.py:13-40, timing.py:58-150) and the
median filter (timing.py:19-55, triton_ops.py:43-109). The CPU restatement in
oracle/timing_oracle.py is pinned by brute force over all monotone paths,
hand-derived tie cases, agreement with the reference's CPU variant on tie-free
inputs and numpy's median; on the GPU the HIP kernels must match it exactly."""
import numpy as np
import pytest
import torch

from oracle import timing_oracle as T


def brute_min_path(x):
    """Minimum over all monotone paths (steps down, right, diagonal) from (0,0) to
    (M-1,N-1) of the summed costs, by exhaustive recursion (tiny inputs)."""
    M, N = x.shape
    best = {}

    def go(i, j):
        if (i, j) in best:
            return best[(i, j)]
        if i == 0 and j == 0:
            v = np.float64(x[0, 0])
        else:
            cands = []
            if i > 0 and j > 0:
                cands.append(go(i - 1, j - 1))
            if i > 0:
                cands.append(go(i - 1, j))
            if j > 0:
                cands.append(go(i, j - 1))
            v = x[i, j] + min(cands)
        best[(i, j)] = v
        return v

    return go(M - 1, N - 1)


@pytest.mark.parametrize("shape", [(1, 1), (1, 4), (4, 1), (3, 5), (5, 4), (6, 6)])
def test_dtw_oracle_is_the_minimum_path(shape):
    rng = np.random.default_rng(sum(shape))
    x = rng.integers(0, 9, size=shape).astype(np.float32)  # small integers: exact sums
    cost, trace = T.dtw_trace(x)
    assert cost[-1, -1] == brute_min_path(x.astype(np.float64))
    path = T.backtrace(trace)
    # the path starts at (0,0), ends at (M-1,N-1), moves by unit steps and costs the minimum
    assert tuple(path[:, 0]) == (0, 0) and tuple(path[:, -1]) == (shape[0] - 1, shape[1] - 1)
    steps = np.diff(path, axis=1)
    assert set(map(tuple, steps.T)) <= {(1, 1), (1, 0), (0, 1)}
    assert x[path[0], path[1]].sum() == cost[-1, -1]


def test_dtw_tie_order():
    # all-equal costs: at (1,1) only the diagonal is finite -> 0; at (1,2): c0 = inf, c1 = inf,
    # c2 = cost[1,1] -> 2; at (2,2): c0 = 1, c1 = 2, c2 = 2 -> 0; a 2x2 tie c0 = c1 picks 0
    x = np.ones((2, 2), np.float32)
    cost, trace = T.dtw_trace(x)
    assert trace[1, 1] == 0 and trace[1, 2] == 2 and trace[2, 1] == 1 and trace[2, 2] == 0
    # c1 == c2 < c0 -> 1 (the reference kernel's store order), the CPU variant gives 2
    x = np.array([[9, -3], [-3, 5]], np.float32)
    cost, trace = T.dtw_trace(x)
    assert cost[1, 1] == 9 and cost[1, 2] == 6 and cost[2, 1] == 6
    assert trace[2, 2] == 1 and cost[2, 2] == 11
    _, tc = T.dtw_trace_cpu(x)
    assert tc[2, 2] == 2
    y = np.array([[0, 0, 0], [0, 0, 0], [0, 0, 0]], np.float32)
    _, ty = T.dtw_trace(y)
    _, tc = T.dtw_trace_cpu(y)
    # interior cells see three equal predecessors: 0 here, 2 in the CPU variant; the first
    # row and column see one finite predecessor and agree (2 and 1)
    assert (ty[2:, 2:] == 0).all() and (tc[2:, 2:] == 2).all()
    assert (ty[1, 2:] == 2).all() and (tc[1, 2:] == 2).all()
    assert (ty[2:, 1] == 1).all() and (tc[2:, 1] == 1).all()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_dtw_oracle_agrees_with_cpu_variant_without_ties(seed):
    rng = np.random.default_rng(seed)
    x = rng.random((13, 29)).astype(np.float32)
    c1, t1 = T.dtw_trace(x)
    c2, t2 = T.dtw_trace_cpu(x)
    assert np.array_equal(c1, c2) and np.array_equal(t1, t2)


def test_median_oracle():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4, 37)).astype(np.float32)
    for w in (1, 3, 7, 11):
        p = w // 2
        got = T.median_filter(x, w)
        xp = np.pad(x, [(0, 0), (0, 0), (p, p)], mode="reflect")
        want = np.stack([np.median(xp[..., t:t + w], axis=-1) for t in range(37)], -1)
        assert np.array_equal(got, want.astype(np.float32)), w
    # known answer, reflect padding: [1, 5, 2, 8, 3] width 3 -> pads [5 | ... | 8]
    assert T.median_filter(np.array([1, 5, 2, 8, 3], np.float32), 3).tolist() == [5, 2, 5, 3, 8]
    # too short a row is returned unchanged
    s = np.array([[1.0, 2.0]], np.float32)
    assert T.median_filter(s, 7) is s


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("shape,kind", [((1, 1), "rand"), ((1, 50), "rand"), ((30, 1), "rand"),
                                        ((57, 300), "rand"), ((448, 1500), "rand"), ((1023, 200), "rand"),
                                        ((40, 90), "ties"), ((25, 60), "inf")])
def test_dtw_matches_oracle(iw, gpu, shape, kind):
    print("dtw", shape, kind, flush=True)
    from importlib import import_module

    tm = import_module(iw.__name__ + ".timing")
    rng = np.random.default_rng(shape[0] * 7 + shape[1])
    if kind == "ties":
        x = rng.integers(0, 3, size=shape).astype(np.float32)
    else:
        x = rng.standard_normal(shape).astype(np.float32)
    if kind == "inf":
        x[rng.random(shape) < 0.1] = np.inf
    cost, trace = T.dtw_trace(x)
    got = tm.dtw_trace(torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(got, trace)
    assert np.array_equal(tm.dtw(torch.from_numpy(x).cuda()), T.backtrace(trace))


@pytest.mark.gpu
@pytest.mark.parametrize("shape,w", [((8, 100), 7), ((2, 3, 1500), 7), ((5, 4), 3), ((1, 64), 1), ((6, 333), 31),
                                     ((3, 16), 15)])
def test_median_filter_matches_oracle(iw, gpu, shape, w):
    print("median", shape, w, flush=True)
    from importlib import import_module

    tm = import_module(iw.__name__ + ".timing")
    rng = np.random.default_rng(w)
    x = rng.standard_normal(shape).astype(np.float32)
    x[..., ::5] = np.round(x[..., ::5])  # repeated values
    got = tm.median_filter(torch.from_numpy(x).cuda(), w).cpu().numpy()
    assert np.array_equal(got, T.median_filter(x, w))
    short = torch.zeros((2, 3), device="cuda")
    assert tm.median_filter(short, 7) is short
