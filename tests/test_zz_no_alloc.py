"""xnq_qtensor_matmul_t_noalloc: the entry point that allocates nothing (its
scratch is the library's static per-GPU device array) against
xnq_qtensor_matmul_t_ws, the entry point it shares its kernels with, on two
calls in a row, the second with fewer rows, on every route that uses scratch.
Both go through the C ABI.  The bar is bit equality: the same kernels run on
the same inputs with the same split counts."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14
NOALLOC_SCRATCH = 64 << 20


def _pair(qt, m, k, n, x, dev):
    want = torch.full((m, n), float("nan"), device=dev)
    ws = torch.empty(max(qt.matmul_t_workspace_size(m), 1), dtype=torch.uint8, device=dev)
    qt.matmul_t_ws((m, k, n), x, ws, want)
    got = torch.full((m, n), float("nan"), device=dev)
    qt.matmul_t_noalloc((m, k, n), x, got)
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


@pytest.mark.parametrize("dt,k,n,ms", [
    (Q4K, 4096, 14336, (512, 300)),   # tiled prefill (row-tiled activation image)
    (Q6K, 4096, 4096, (300, 70)),     # tiled prefill with split-K partials
    (Q4K, 4096, 4096, (64, 16)),      # skinny, split-K partials
    (Q6K, 14336, 4096, (16, 2)),      # skinny, then matvec after quantize
    (Q4K, 14336, 4096, (8, 1)),       # matvec after quantize (m = 1 on this size too)
    (Q4_0, 4096, 14336, (4, 1)),      # 32-element blocks; m = 1 on the fused route
    (Q8_0, 2048, 3000, (9, 3)),
])
def test_noalloc_matches_ws(orc, dev, dt, k, n, ms):
    from xn_amd import GgmlDType, QTensor

    g = torch.Generator(device=dev).manual_seed(299792458 + dt + k + n)
    w = torch.randn((n, k), generator=g, device=dev) * 0.02
    qt = QTensor.quantize_f32(w, (n, k), GgmlDType(dt))
    del w
    for i, m in enumerate(ms):
        x = torch.randn((m, k), generator=g, device=dev)
        got, want = _pair(qt, m, k, n, x, dev)
        assert not np.isnan(got).any(), f"call {i} m={m}: output not fully written"
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {i} m={m} differs from matmul_t_ws"
    if dt == Q4K and n == 4096:
        # and against the oracle once, for the route table's sake
        xh = np.random.default_rng(5).normal(0, 1, (16, k)).astype(np.float32)
        y = torch.empty((16, n), device=dev)
        qt.matmul_t_noalloc((16, k, n), torch.from_numpy(xh).to(dev), y)
        blocks = np.frombuffer(qt.data(), np.uint8)
        from tests.test_gpu_parity import assert_close
        assert_close(y.cpu().numpy(), orc.matmul(Q4K, xh, blocks, n), "noalloc vs oracle")


def test_noalloc_rejects_oversized(dev):
    from xn_amd import GgmlDType, QTensor, XnqError

    k, n = 4096, 256
    qt = QTensor.quantize_f32(torch.zeros((n, k), device=dev), (n, k), GgmlDType.Q4K)
    m = 8192
    assert qt.matmul_t_workspace_size(m) > NOALLOC_SCRATCH
    x = torch.zeros((m, k), device=dev)
    y = torch.zeros((m, n), device=dev)
    with pytest.raises(XnqError, match="scratch"):
        qt.matmul_t_noalloc((m, k, n), x, y)
    # a large m that fits still runs
    m = 2048
    assert qt.matmul_t_workspace_size(m) <= NOALLOC_SCRATCH
    qt.matmul_t_noalloc((m, k, n), x[:m], y[:m])
    torch.cuda.synchronize()
    assert torch.count_nonzero(y[:m]).item() == 0
