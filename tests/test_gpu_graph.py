"""HIP-graph capture of the dense ops (reference tests/test_cuda_graph.py:70-97,
there with an all-zero (8,16,2) trellis that the gfx950 ops refuse as a K=1/8
pack; here with valid packs).

One graph holds exl3_gemv (balanced kernel at m=1, k-split kernel at m=4),
exl3_gemm (MFMA path at m=100), exl3_linear (3INST), dequant_trellis,
p2b_gemv_batched, exl3_gate_up_swiglu (GEMV, narrow MFMA with and without the
split-out finish launch, wide tiles on mul1 raw entries), exl3_fat_gemm and
exl3_fat_gemm_scatter.  It is replayed several times, with new inputs copied
into the captured input tensors and eager calls of the same ops on the same
stream between replays; every replay must equal the eager result on the same
inputs: bit for bit where a kernel sums in a fixed order, within the parity bar
for the fp32-atomic fat kernels (whose summation order varies)."""

import numpy as np
import pytest
import torch

from gpu_util import check_close, make_weight, make_x
from sglang_exl3 import ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _registered():
    ops.register_custom_ops()


def _w(k, n, K, seed):
    tr, su, sv = make_weight(k, n, K, seed)
    sv = (sv.astype(np.float32) * (4.0 / np.sqrt(k))).astype(np.float16)
    return [torch.from_numpy(a).cuda() for a in (tr, su, sv)]


def test_dense_ops_graph_capture_replay():
    k, n, K = 512, 384, 3
    tr, su, sv = _w(k, n, K, 1)
    tr0, su0, sv0 = _w(k, n, 4, 2)                     # 3INST linear
    trg, _, svg = _w(k, n, K, 3)                       # gate/up pair sharing su
    tru, _, svu = _w(k, n, K, 4)
    ptr = lambda *ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device="cuda")
    tabs = (ptr(tr, trg), ptr(su, su), ptr(sv, svg))
    ids = torch.tensor([1, 0], dtype=torch.int32, device="cuda")
    tok = torch.randperm(64, generator=torch.Generator().manual_seed(0))[:48].cuda()
    rw = (torch.rand(48, generator=torch.Generator().manual_seed(1)) + 0.5).to(torch.float16).cuda()

    xs = {m: torch.zeros((m, k), dtype=torch.float16, device="cuda") for m in (1, 2, 4, 16, 48, 100, 200)}
    fat_out = torch.zeros((48, n), dtype=torch.float32, device="cuda")
    scat_out = torch.zeros((64, n), dtype=torch.float32, device="cuda")

    def run():
        o = {}
        o["gemv1"] = torch.ops.sglang_exl3.exl3_gemv(xs[1], tr, su, sv, K, True)
        o["gemv4"] = torch.ops.sglang_exl3.exl3_gemv(xs[4], tr, su, sv, K, False)
        o["gemm100"] = torch.ops.sglang_exl3.exl3_gemm(xs[100], tr, su, sv, K, True)
        o["lin3inst"] = torch.ops.sglang_exl3.exl3_linear(xs[2], tr0, su0, sv0, 4, 0)
        o["dequant"] = torch.ops.sglang_exl3.dequant_trellis(tr, su, sv, K, True)
        o["batched"] = torch.ops.sglang_exl3.p2b_gemv_batched(xs[2], *tabs, ids, K, True, n)
        o["gu2"] = torch.ops.sglang_exl3.exl3_gate_up_swiglu(xs[2], su, trg, svg, tru, svu, K, 1)
        o["gu100"] = torch.ops.sglang_exl3.exl3_gate_up_swiglu(xs[100], su, trg, svg, tru, svu, K, 2, 4.0)
        # 16 rows: the split-out finish launch; 200 rows: wide tiles with mul1 raw entries
        o["gu16"] = torch.ops.sglang_exl3.exl3_gate_up_swiglu(xs[16], su, trg, svg, tru, svu, K, 2)
        o["gu200"] = torch.ops.sglang_exl3.exl3_gate_up_swiglu(xs[200], su, trg, svg, tru, svu, K, 2)
        fat_out.zero_()
        torch.ops.sglang_exl3.exl3_fat_gemm(xs[48], tr, fat_out, sv, K, True, False)
        scat_out.zero_()
        torch.ops.sglang_exl3.exl3_fat_gemm_scatter(xs[48], tr, scat_out, sv, tok, rw, K, False, True)
        o["fat"] = fat_out.clone()
        o["scatter"] = scat_out.clone()
        return o

    def fill(seed):
        for m, x in xs.items():
            x.copy_(torch.from_numpy(make_x(m, k, seed=seed * 10 + m)))

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fill(0)
        run()  # warm-up: sizes every workspace outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            static = run()
        torch.cuda.synchronize()
        for r in range(1, 5):
            print(f"case: dense graph replay {r}", flush=True)
            fill(r)
            g.replay()
            torch.cuda.synchronize()
            got = {name: t.clone() for name, t in static.items()}
            eager = run()  # eager calls on the same stream between replays
            torch.cuda.synchronize()
            for name in got:
                assert got[name].shape == eager[name].shape, name
                if name in ("fat", "scatter"):
                    check_close(got[name].cpu().numpy(), eager[name].cpu().numpy(), f"graph {name} replay {r}")
                else:
                    assert torch.equal(got[name], eager[name]), f"graph replay {r}: {name} differs from eager"
            assert float(got["gemv1"].float().abs().sum()) > 0
