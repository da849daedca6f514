"""rq_matmul_many_noalloc: rq_matmul_many with its m >= 2 Q8_1 scratch in the
library's fixed device array (no allocation). Its outputs must equal
rq_matmul_many's bit for bit (same kernels, same quantization), on calls in a
row whose inputs shrink (the array keeps the previous call's contents), in
both kernel families; sizes over the array's capacity are refused."""
import numpy as np
import pytest
import torch

from gpu_util import make_weight, upload
from rllm_amd import _lib
from rllm_amd.errors import ShapeError

pytestmark = pytest.mark.gpu


def _run(gpu, fn, x, ws, m):
    outs = [gpu.alloc(m * w.rows) for w in ws]
    fn(x, ws, outs, m)
    return [gpu.to_host(o, m * w.rows).copy() for o, w in zip(outs, ws)]


@pytest.mark.parametrize("family", ["dot4", "mfma"])
def test_noalloc_matches_matmul_many(gpu, orc, family):
    gpu.set_kernels(family)
    try:
        # Calls in a row, each smaller than the one before: (k, m, weights).
        plan = [(4096, 12, [(12, 256), (12, 64), (14, 64)]),
                (4096, 5, [(12, 256)]),
                (1024, 3, [(8, 96), (2, 64)]),
                (512, 2, [(14, 32)]),
                (4096, 1, [(12, 256), (14, 64)])]
        for i, (k, m, spec) in enumerate(plan):
            ws = [upload(gpu, t, make_weight(orc, t, n, k, 300 + 10 * i + j, "normal"), n, k)
                  for j, (t, n) in enumerate(spec)]
            x = gpu.from_host(orc.normal(400 + i, m * k))
            want = _run(gpu, gpu.matmul_many, x, ws, m)
            got = _run(gpu, gpu.matmul_many_noalloc, x, ws, m)
            for a, b in zip(got, want):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {i} (k={k}, m={m}) differs"
            # and against the int8 oracle
            qs, d, _ = orc.quantize_q8_1(gpu.to_host(x), m, k)
            for (t, n), w, a in zip(spec, ws, got):
                wb = gpu.weight_to_gguf(w)
                orc.assert_close(f"noalloc call {i}", orc.matvec_q8_1(t, wb, n, k, qs, d, m), a, 1e-3)
            del ws
    finally:
        gpu.set_kernels("auto")


def test_noalloc_capacity(gpu, orc):
    k, n = 4096, 32
    w = upload(gpu, 12, make_weight(orc, 12, n, k, 7, "normal"), n, k)
    m = _lib.NOALLOC_MAX_VALUES // k  # exactly at capacity: accepted
    x = gpu.from_host(orc.normal(8, (m + 1) * k))
    out = gpu.alloc((m + 1) * n)
    gpu.matmul_many_noalloc(x, [w], [out], m)
    want = gpu.alloc(m * n)
    gpu.matmul_many(x, [w], [want], m)
    assert torch.equal(out[:m * n].view(torch.int32), want.view(torch.int32))
    with pytest.raises(ShapeError, match="fixed scratch"):
        gpu.matmul_many_noalloc(x, [w], [out], m + 1)
