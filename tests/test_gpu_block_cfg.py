"""A block forward that alternates text lengths, as the engine's CFG loop
does (src/core/engine.cpp:319-330 runs the DiT on the positive, then the
negative text embedding: 58 and 64 tokens in the bundled
embeddings/default_{pos,neg}_emb.bin).

The block's RoPE table depends on the rope mode and frequencies alone and
only grows, so after one forward at each length the forwards enqueue kernels
only: no table rebuild, no host wait.  Checked here:
  * every alternating forward is bit-identical to a fresh block's forward at
    that length;
  * the second pair of forwards, with a caller workspace, captures in a HIP
    graph (torch.cuda.graph fails on a stream synchronisation or an
    allocation inside the capture), and three replays, each after eager work
    on the same block, reproduce the eager outputs bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import ncnn_files as nf

pytestmark = pytest.mark.gpu

DIM, HEADS, MLP = 256, 2, 512
T, H, W = 2, 6, 10
LENGTHS = (58, 64)


def _block(hip, rng_seed, dtype):
    rng = np.random.default_rng(rng_seed)
    w = nf.random_weights(rng, DIM, MLP, shared=False)
    cfg = hip.block_config(dim=DIM, heads=HEADS, mlp_hidden=MLP, shifted_window=1)
    blk = hip.DitBlock.from_host(cfg, w, dtype)
    blk.set_runtime_shape(T, H, W)
    return blk, w


@pytest.mark.parametrize("dtype_name", ["f16", "f32"])
def test_cfg_alternating_text_lengths(hip, device, dtype_name):
    dtype = hip.F16 if dtype_name == "f16" else hip.F32
    td = torch.float16 if dtype == hip.F16 else torch.float32
    print(f"[cfg] block dim={DIM} heads={HEADS} grid {T}x{H}x{W} lengths {LENGTHS} dtype={dtype_name}", flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(11)
    vid = torch.randn((T * H * W, DIM), generator=g, device=device).to(td)
    txts = {L: torch.randn((L, DIM), generator=g, device=device).to(td) for L in LENGTHS}
    emb = torch.randn((6 * DIM,), generator=g, device=device)

    def run(blk, L, ws=None, outs=None, stream=None):
        ov, ot = outs if outs is not None else (torch.empty_like(vid), torch.empty_like(txts[L]))
        blk.forward(vid, txts[L], emb, ov, ot, workspace=ws, stream=stream)
        return ov, ot

    # fresh blocks, one per length
    ref = {}
    for L in LENGTHS:
        blk, _ = _block(hip, 3, dtype)
        ov, ot = run(blk, L)
        torch.cuda.synchronize()
        ref[L] = (ov.clone(), ot.clone())
        blk.close()

    blk, _ = _block(hip, 3, dtype)
    ws = torch.empty(max(blk.workspace_size(L) for L in LENGTHS), dtype=torch.uint8, device=device)
    # eager, alternating as the CFG loop does
    for rep in range(2):
        for L in LENGTHS:
            ov, ot = run(blk, L, ws)
            torch.cuda.synchronize()
            assert torch.equal(ov, ref[L][0]) and torch.equal(ot, ref[L][1]), (rep, L)

    if dtype == hip.F32:
        blk.close()
        return
    # the next pair in a HIP graph, then three replays
    outs = {L: (torch.empty_like(vid), torch.empty_like(txts[L])) for L in LENGTHS}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for L in LENGTHS:
                run(blk, L, ws, outs[L], stream=torch.cuda.current_stream())
    torch.cuda.current_stream().wait_stream(side)
    for replay in range(3):
        for L in outs:
            outs[L][0].fill_(float("nan"))
            outs[L][1].fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for L in LENGTHS:
            assert torch.equal(outs[L][0], ref[L][0]) and torch.equal(outs[L][1], ref[L][1]), (replay, L)
        # eager work on the same block between replays
        ov, ot = run(blk, LENGTHS[replay % 2], ws)
        torch.cuda.synchronize()
        assert torch.equal(ov, ref[LENGTHS[replay % 2]][0])
    del graph
    blk.close()
