"""The no-allocation entry point slhip_dual_matvec_int8_noalloc against the workspace form slhip_dual_matvec_int8
(the same kernels: bit-identical results), on two calls in a row, the second smaller, and its size limit."""
import numpy as np
import pytest

from sharplight_amd import native, synth
from tests.devutil import Dev, log

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("first,second", [(("q4_k", 8, 4096, 1024), ("q6_k", 2, 2048, 512))])
def test_noalloc_matches_workspace_form(device, first, second):
    for fmt, T, K, N in (first, second):
        wg = synth.quant_table(fmt, N, K, seed=50, tid=1)
        wu = synth.quant_table(fmt, N, K, seed=50, tid=2)
        x = synth.normal(50, 3, (T, K))
        with Dev() as d:
            px, pg, pu = d.put(x), d.put(wg), d.put(wu)
            y1, y2 = d.empty(T * N * 4), d.empty(T * N * 4)
            work = d.empty(T * native.q8_row_bytes(K))
            log(f"dual_matvec_int8 workspace fmt={fmt} T={T} K={K} N={N}")
            native.dual_matvec_int8("silu", fmt, "f32", "f32", px, T, K, pg, pu, N, y1, work, T * native.q8_row_bytes(K))
            log(f"dual_matvec_int8_noalloc fmt={fmt} T={T} K={K} N={N}")
            native.dual_matvec_int8_noalloc("silu", fmt, "f32", "f32", px, T, K, pg, pu, N, y2)
            native.synchronize()
            a = d.get(y1, (T, N), np.float32)
            b = d.get(y2, (T, N), np.float32)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (fmt, T, K, N)


def test_noalloc_size_limit_and_small_workspace(device):
    with Dev() as d:
        p = d.empty(4096)
        with pytest.raises(native.SlhipNotSupported, match="static"):
            native.dual_matvec_int8_noalloc("silu", "q4_k", "f32", "f32", p, 64, 16384, p, p, 16, p)
        with pytest.raises(native.SlhipArgumentError, match="workspace"):
            native.dual_matvec_int8("silu", "q4_k", "f32", "f32", p, 2, 4096, p, p, 16, p, p, 100)
        native.dual_matvec_int8_noalloc("silu", "q4_k", "f32", "f32", None, 0, 4096, None, None, 16, None)
