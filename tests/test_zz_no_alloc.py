"""strata_gemvn_noalloc (no counterpart in the reference; for callers that cannot allocate) through the C ABI: the same
bits as strata_gemvn on two calls in a row, the second smaller, and requests past its fixed scratch rejected."""
import numpy as np
import pytest

import rustingstrata_amd as S
from rustingstrata_amd import ggml
from tests.helpers import normal, random_blocks

pytestmark = pytest.mark.gpu


def run(hip, fn, ty, rows, cols, nt, seed):
    w = random_blocks(ty, rows, cols, seed=seed)
    t = hip.upload_tensor(ty, w)
    x = hip.upload(normal((nt, cols), seed=seed + 1))
    y = hip.alloc(nt * rows * 4)
    getattr(hip, fn)(t, x, cols, y, rows, nt)
    return hip.get(y, np.float32, nt * rows)


@pytest.mark.parametrize("ty", [ggml.Q4_K, ggml.Q6_K, ggml.Q8_0])
def test_gemvn_noalloc_matches_gemvn(hip, ty):
    # first call: the largest request the fixed scratch holds (4 inputs of 16384 values); then a smaller one, whose
    # scales land where the first call's int8 values were
    for rows, cols, nt, seed in [(300, 16384, 4, 11), (129, 2048, 3, 12), (64, 4096, 1, 13)]:
        a = run(hip, "gemvn_noalloc", ty, rows, cols, nt, seed + ty)
        b = run(hip, "gemvn", ty, rows, cols, nt, seed + ty)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rows, cols, nt, int((a != b).sum()))


def test_gemvn_noalloc_rejects(hip):
    w = random_blocks(ggml.Q4_K, 4, 256 * 65, seed=1)
    t = hip.upload_tensor(ggml.Q4_K, w)
    x, y = hip.alloc(5 * 256 * 65 * 4), hip.alloc(5 * 4 * 4)
    with pytest.raises(S.StrataError, match="at most 16384"):
        hip.gemvn_noalloc(t, x, 256 * 65, y, 4, 2)
    t2 = hip.upload_tensor(ggml.Q4_K, random_blocks(ggml.Q4_K, 4, 256, seed=2))
    with pytest.raises(S.StrataError, match=r"gemvn: 5 inputs \(1 to 4\)"):
        hip.gemvn_noalloc(t2, x, 256, y, 4, 5)
