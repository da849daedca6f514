"""rq_matmul_many_noalloc: rq_matmul_many with its m >= 2 Q8_1 scratch in the
library's fixed device array (no allocation). Its outputs must equal
rq_matmul_many's bit for bit (same kernels, same quantization), on calls in a
row whose inputs shrink (the array keeps the previous call's contents), in
both kernel families; sizes over the array's capacity are refused. It never
takes the f16 GEMM route, so at 65 columns and more it is compared with
rq_matmul_many held to the int8 path (rq_set_gemm_min_m 0)."""
import numpy as np
import pytest
import torch

from gpu_util import make_weight, upload
from rllm_amd import _lib
from rllm_amd.backend import GEMM_MIN_M_DEFAULT
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
    gpu.set_gemm_min_m(0)
    try:
        gpu.matmul_many(x, [w], [want], m)
    finally:
        gpu.set_gemm_min_m(GEMM_MIN_M_DEFAULT)
    assert torch.equal(out[:m * n].view(torch.int32), want.view(torch.int32))
    with pytest.raises(ShapeError, match="fixed scratch"):
        gpu.matmul_many_noalloc(x, [w], [out], m + 1)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
@pytest.mark.parametrize("family", ["dot4", "mfma"])
def test_noalloc_under_capture_on_a_fresh_context(orc, family):
    """What the entry point is for: on a context that has never allocated
    scratch (no rq_reserve, no earlier m >= 2 call), rq_matmul_many_noalloc
    at m >= 2 records into a HIP graph, where rq_matmul_many's scratch growth
    is refused, and every replay equals an eager call bit for bit. Device
    memory that the library could have taken does not change."""
    from rllm_amd.backend import HipBackend

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    fresh = HipBackend(0)
    try:
        fresh.set_kernels(family)
        k, m = 4096, 6
        spec = [(12, 128), (12, 64), (14, 64)]
        ws = [upload(fresh, t, make_weight(orc, t, n, k, 700 + i, "normal"), n, k) for i, (t, n) in enumerate(spec)]
        x = fresh.from_host(orc.normal(710, m * k))
        g_outs = [fresh.alloc(m * n) for _, n in spec]
        # rq_matmul_many would have to grow the context's scratch: refused.
        with pytest.raises(ShapeError, match="rq_reserve"):
            _capture(fresh, lambda: fresh.matmul_many(x, ws, g_outs, m))
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info(fresh.device)
        g = _capture(fresh, lambda: fresh.matmul_many_noalloc(x, ws, g_outs, m))
        for rep in range(3):
            x.copy_(torch.from_numpy(orc.normal(720 + rep, m * k)).to(fresh.device))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = [o.clone() for o in g_outs]
            want = _run(fresh, fresh.matmul_many_noalloc, x, ws, m)
            for a, b in zip(got, want):
                assert np.array_equal(a.cpu().numpy().view(np.uint32), b.view(np.uint32)), f"replay {rep} differs"
        free1, _ = torch.cuda.mem_get_info(fresh.device)
        # torch's own graph pool may take a few MiB; the library's scratch for
        # this call (m * k codes + scales) would be in addition, and is not.
        assert free0 - free1 < (64 << 20), f"device memory dropped by {(free0 - free1) >> 20} MiB"
        # and the last replay equals rq_matmul_many (which now grows its scratch)
        want = _run(fresh, fresh.matmul_many, x, ws, m)
        for a, b in zip(got, want):
            assert np.array_equal(a.cpu().numpy().view(np.uint32), b.view(np.uint32)), "noalloc != matmul_many"
        del g
    finally:
        fresh.synchronize()
        fresh.close()


def _capture(gpu, fn):
    s = torch.cuda.Stream(gpu.device)
    main = torch.cuda.current_stream(gpu.device)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    gpu.set_stream(s)
    try:
        with torch.cuda.graph(g, stream=s):
            fn()
    finally:
        gpu.set_stream(main)
    return g
