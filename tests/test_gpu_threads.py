"""Two host threads launch through the C ABI at once, each on its own HIP
stream (default priority): the launch paths' per-device caches, once-per-
device kernel attributes and the tuning table are shared state, so the
results of every call must be bit-identical to the same calls made from one
thread."""
import threading

import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def test_two_host_threads_two_streams():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    print("[case] two host threads, two streams: gemv 17408x5120, gemm 5120x6144x8 and x300", flush=True)
    B.lib()
    jobs = []
    for k, (n_out, n_in, n_tok) in enumerate([(17408, 5120, 1), (5120, 6144, 8), (1000, 5120, 300)]):
        W = torch.from_numpy(O.gen_weights(7000 + k, n_out, n_in)).cuda()
        X = np.stack([O.fwht(O.gen_normal(7010 + k + t, n_in)) for t in range(n_tok)])
        Xq = torch.from_numpy(O.quantize_chunk_major(X)).cuda()
        jobs.append((W, Xq, n_out, n_in, n_tok))

    def run(job, stream):
        W, Xq, n_out, n_in, n_tok = job
        Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
        B.gemm(W, Xq, Y, n_out, n_in, n_tok, stream=stream)
        return Y

    ref = [run(j, None) for j in jobs]
    torch.cuda.synchronize()
    ref = [r.cpu().numpy() for r in ref]

    results, errors = {}, []

    def worker(tid):
        try:
            s = torch.cuda.Stream()
            outs = []
            with torch.cuda.stream(s):
                for it in range(12):
                    j = (tid + it) % len(jobs)
                    outs.append((j, run(jobs[j], s)))
                    if it % 5 == 0:
                        B.reload_tuning()
            s.synchronize()
            results[tid] = [(j, y.cpu().numpy()) for j, y in outs]
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    ts = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    for tid in range(2):
        assert len(results[tid]) == 12
        for j, y in results[tid]:
            np.testing.assert_array_equal(y.view(np.uint32), ref[j].view(np.uint32))
