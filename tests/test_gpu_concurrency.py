"""One quantized weight used from several host threads and streams at once.

xn's QuantizedType is Send + Sync (mod.rs:199) and a QTensor is shared by
every caller of a model.  Here four host threads, each on its own HIP
stream, call matmul_t on the same qtensors concurrently with inputs that take
every route (m = 1 fused decode, m = 4 matvec, m = 16 skinny MFMA, m = 300
tiled MFMA), plus the grouped and SiLU-gated entries.  The kernels are
deterministic, so every concurrent result must equal the one the same call
gives alone, bit for bit."""
import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_concurrent_matmul_t_on_shared_weights(dev):
    from xn_amd import GgmlDType, QTensor
    from xn_amd.quantized import matmul_t_group, matmul_t_silu_gate

    g = torch.Generator(device=dev).manual_seed(77)
    k, n = 1024, 768
    qa = QTensor.quantize_f32(torch.randn((n, k), generator=g, device=dev) * 0.02, (n, k), GgmlDType.Q4K)
    qb = QTensor.quantize_f32(torch.randn((n, k), generator=g, device=dev) * 0.02, (n, k), GgmlDType.Q4K)
    q6 = QTensor.quantize_f32(torch.randn((n, k), generator=g, device=dev) * 0.02, (n, k), GgmlDType.Q6K)
    ms = [1, 4, 16, 300]
    xs = {m: torch.randn((m, k), generator=g, device=dev) for m in ms}

    def calls(m, outs):
        qa.matmul_t((m, k, n), xs[m], outs["a"])
        q6.matmul_t((m, k, n), xs[m], outs["6"])
        matmul_t_silu_gate(qa, qb, (m, k, n), xs[m], outs["gate"])
        matmul_t_group([qa, qb], m, k, xs[m], [outs["ga"], outs["gb"]])

    def fresh(m):
        return {key: torch.full((m, n), float("nan"), device=dev) for key in ("a", "6", "gate", "ga", "gb")}

    want = {}
    for m in ms:
        want[m] = fresh(m)
        calls(m, want[m])
    torch.cuda.synchronize()

    nthreads, reps = 4, 6
    got = [[None] * reps for _ in range(nthreads)]
    errors = []
    start = threading.Barrier(nthreads)

    def worker(t):
        try:
            s = torch.cuda.Stream(dev)
            start.wait()
            with torch.cuda.stream(s):
                for r in range(reps):
                    m = ms[(t + r) % len(ms)]
                    outs = fresh(m)
                    calls(m, outs)
                    got[t][r] = (m, outs)
            s.synchronize()
        except Exception as e:  # surfaced below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nthreads)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for t in range(nthreads):
        for r in range(reps):
            m, outs = got[t][r]
            for key, y in outs.items():
                assert torch.equal(y, want[m][key]), f"thread {t} rep {r} m={m} {key}"
