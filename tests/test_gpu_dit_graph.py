"""A whole DiT forward (input head, 32 blocks, output head; src/model/dit.cpp:
281-383) captured in a HIP graph.  With the caller's workspace and the
blocks' RoPE tables grown by an eager forward at the same shape, a forward
only enqueues kernels and device copies: torch.cuda.graph fails on a host
synchronisation or an allocation inside the capture.  Three replays, each
followed by an eager forward at another text length (the CFG loop
alternates the positive and negative texts, src/core/engine.cpp:319-330),
must each equal the eager result bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from test_gpu_dit import SMALL, build_dit, dev, small_dit_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_dit_forward_in_a_graph(hip, device, dtype):
    code = hip.F32 if dtype == "f32" else hip.F16
    print(f"[dit graph] {dtype}", flush=True)
    wi, blocks_w, wo = small_dit_weights(71)
    rng = np.random.default_rng(72)
    T, H, W = 2, 8, 12
    lengths = (9, 12)
    latent = dev(rng.standard_normal((33, T, H, W), dtype=np.float32))
    texts = {L: dev(rng.standard_normal((L, SMALL["text_channels"]), dtype=np.float32)) for L in lengths}
    dit = build_dit(hip, wi, blocks_w, wo, code)
    try:
        ws = torch.empty(max(dit.workspace_size(T, H, W, L) for L in lengths), dtype=torch.uint8, device=device)

        def run(L, out=None, stream=None):
            out = torch.full((16, T, H, W), float("nan"), device=device) if out is None else out
            dit.forward(latent, texts[L], 1000.0, out, workspace=ws, stream=stream)
            return out

        ref = {}
        for L in lengths:
            ref[L] = run(L)
        torch.cuda.synchronize()
        for L in lengths:
            assert torch.isfinite(ref[L]).all(), L

        outs = {L: torch.empty((16, T, H, W), device=device) for L in lengths}
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for L in lengths:
                    run(L, outs[L], stream=torch.cuda.current_stream())
        torch.cuda.current_stream().wait_stream(side)
        for replay in range(3):
            for L in lengths:
                outs[L].fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            for L in lengths:
                assert torch.equal(outs[L], ref[L]), (replay, L)
            eager = run(lengths[replay % 2])
            torch.cuda.synchronize()
            assert torch.equal(eager, ref[lengths[replay % 2]]), replay
        del graph
    finally:
        dit.close()
