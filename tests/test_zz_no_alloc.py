"""hero_argmax_noalloc (partial keys in a static device array, no allocation)
against hero_argmax (caller-provided scratch) through the C ABI: two calls in a
row on one GPU, the second with fewer rows and a shorter vocabulary, so the
array still holds the first call's keys when the second runs."""
import numpy as np
import pytest

from gpu_util import check, dev, empty, host, ptr, stream

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    import torch

    from hero_amd._lib import lib as _lib

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return _lib


def logits_with_ties(rng, m, n):
    x = rng.standard_normal((m, n)).astype(np.float32)
    x[0, [n - 1, min(7, n - 2), n // 2]] = 40.0  # tie: the lowest index wins
    x[1 % m, :] = -3.0
    x[1 % m, n // 3] = 0.0
    x[1 % m, 2] = -0.0                     # -0 ties +0
    x[m - 1, n - 1] = 50.0                 # last element
    return x


@pytest.mark.parametrize("first,second", [((40, 151936), (3, 1000)), ((64, 32000), (1, 5))])
def test_noalloc_argmax_equals_argmax_on_two_calls(lib, first, second):
    from hero_amd._lib import HERO_EINVAL

    rng = np.random.default_rng(first[0] + second[1])
    for m, n in (first, second):
        x = logits_with_ties(rng, m, n)
        d_x = dev(x)
        out_a, out_b = empty(m * 4), empty(m * 4)
        scratch = empty(m * 128 * 8)
        check(lib.hero_argmax(ptr(d_x), m, n, ptr(out_a), ptr(scratch), stream()))
        check(lib.hero_argmax_noalloc(ptr(d_x), m, n, ptr(out_b), stream()))
        a, b = host(out_a, np.int32), host(out_b, np.int32)
        assert np.array_equal(a, b), f"m={m} n={n}"
        assert list(b) == [int(np.argmax(r)) for r in x]
    assert lib.hero_argmax_noalloc(ptr(d_x), 65, 16, ptr(out_b), stream()) == HERO_EINVAL


def test_noalloc_argmax_under_graph_capture(lib):
    """hero_argmax_noalloc recorded into a HIP graph (its documented use: the
    scratch address is resolved by an eager call first) and replayed three
    times over new logits written between the replays, each replay checked
    against hero_argmax run eagerly"""
    import torch

    m, n = 5, 151936
    rng = np.random.default_rng(77)
    d_x = dev(logits_with_ties(rng, m, n))
    out_g, out_e = empty(m * 4), empty(m * 4)
    scratch = empty(m * 128 * 8)
    check(lib.hero_argmax_noalloc(ptr(d_x), m, n, ptr(out_g), stream()))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        check(lib.hero_argmax_noalloc(ptr(d_x), m, n, ptr(out_g), stream()))
    for i in range(3):
        x = logits_with_ties(rng, m, n)
        x[2, rng.integers(0, n)] = 60.0 + i
        d_x.copy_(dev(x))
        g.replay()
        torch.cuda.synchronize()
        check(lib.hero_argmax(ptr(d_x), m, n, ptr(out_e), ptr(scratch), stream()))
        got, ref = host(out_g, np.int32), host(out_e, np.int32)
        assert np.array_equal(got, ref), f"replay {i}: {got} vs {ref}"
        assert list(got) == [int(np.argmax(r)) for r in x]
