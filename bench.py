"""Benchmark of the windowed multimodal attention path on one MI355X.

Workload: the SeedVR2-3B DiT windowed MM-attention at 720p x 21 frames — latent
grid 6x45x80 (21600 video tokens), windows 2x9x16, 20 heads x 128 dims, 58
text tokens attended jointly by every window, fp16 activations N(0,1),
QK-RMSNorm (gamma ~ U(0.5, 1.5)) + RoPE (the reference's mmrope3d).  A step
is one unshifted layer (75 windows) followed by one shifted layer (144 ragged
windows), as consecutive DiT blocks alternate them.  Inputs are resident in
HBM before timing starts.

Prints one JSON line: window-attention TFLOPS of the step (algorithmic flops
sum_w 4 * S_w^2 * 128 * 20 / time), the roofline of the attention launches
(HBM-bound: algorithmic bytes = one read of q/k/v and one write of the
outputs), and the CPU oracle timed on a bounded sample on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
for p in (REPO / "seedvr2-ncnn-valkan_amd", REPO / "tests", REPO / "oracle"):
    sys.path.insert(0, str(p))

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
T, H, W, L_TXT, HEADS, HD = 6, 45, 80, 58, 20, 128
WIN = (2, 9, 16)


def plan_stats(shifted: bool):
    import sv2hip
    wins = sv2hip.window_plan(sv2hip.rule(T, H, W, shifted, *WIN))
    sizes = [(w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) for w in wins]
    flops = sum(4.0 * (v + L_TXT) ** 2 * HD * HEADS for v in sizes)
    return wins, sizes, flops


ATTENTION_SOURCE = REPO / "seedvr2-ncnn-valkan_amd" / "csrc" / "attention.hip"
TRAFFIC_FILE = REPO / "profiles" / "window_attention_720p_traffic.json"


def source_sha256(path: Path = ATTENTION_SOURCE) -> str:
    import hashlib
    return hashlib.sha256(path.read_bytes()).hexdigest()


def measured_traffic():
    """HBM bytes per attention launch from the committed FETCH_SIZE /
    WRITE_SIZE measurement, used only when it measured this kernel source
    (its attention_source_sha256 stamp); else None and the reason."""
    if not TRAFFIC_FILE.exists():
        return None, "no traffic measurement committed"
    try:
        tf = json.loads(TRAFFIC_FILE.read_text())
    except ValueError:
        return None, "traffic file does not parse"
    if tf.get("attention_source_sha256") != source_sha256():
        return None, "traffic file measured another attention kernel source"
    return tf.get("hbm_bytes_per_launch"), "FETCH_SIZE/WRITE_SIZE of this kernel source, " + TRAFFIC_FILE.name


def algorithmic_bytes(elem=2):
    tokens = T * H * W + L_TXT
    return tokens * 3 * HEADS * HD * elem + tokens * HEADS * HD * elem


def host_cpu() -> dict:
    """The host's core count (the cores this process may run on) and CPU model."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": nproc, "cpu_model": model, "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline(target_s: float = 15.0):
    """The CPU oracle on the shifted 720p plan: video queries of a sample of
    windows plus the text queries of every window (the text output averages
    over all windows).  Returns TFLOPS of the work actually done.

    Threads: all cores this process may use, capped by OMP_NUM_THREADS (the
    CPU share a GPU's host process is given, when set) and by the 20 heads the
    oracle's attention parallelises over."""
    import oracle
    from parity import reference_freqs
    host = host_cpu()
    threads = host["nproc"]
    if host["omp_num_threads"]:
        threads = min(threads, int(host["omp_num_threads"]))
    threads = max(1, min(threads, HEADS))
    wins, sizes, _ = plan_stats(True)
    rng = np.random.default_rng(7)
    D = HEADS * HD
    vid = rng.standard_normal((T * H * W, 3 * D), dtype=np.float32).astype(np.float16).astype(np.float32)
    txt = rng.standard_normal((L_TXT, 3 * D), dtype=np.float32).astype(np.float16).astype(np.float32)
    gam = list(rng.uniform(0.5, 1.5, (4, 128)).astype(np.float32))
    freqs = reference_freqs()

    def run(k):
        mask = np.zeros(len(wins), np.uint8)
        mask[np.linspace(0, len(wins) - 1, k).astype(int)] = 1
        work = 0.0
        for wi, v in enumerate(sizes):
            s = v + L_TXT
            queries = (v if mask[wi] else 0) + L_TXT
            work += 4.0 * queries * s * HD * HEADS
        t0 = time.perf_counter()
        oracle.window_attention(vid, txt, T, H, W, heads=HEADS, freqs=freqs, gammas=gam, shifted=True,
                                wt=WIN[0], wh=WIN[1], ww=WIN[2], threads=threads, video_mask=mask)
        return time.perf_counter() - t0, work, int(mask.sum())

    # two-point fit: a fixed cost (text queries of every window) plus a cost
    # per window whose video queries are evaluated
    t_a, _, _ = run(4)
    t_b, _, _ = run(12)
    per_window = max((t_b - t_a) / 8.0, 1e-4)
    fixed = max(t_a - 4 * per_window, 0.0)
    k = int(min(len(wins), max(12, (target_s - fixed) / per_window)))
    dt, work, k = run(k)
    return {
        "value": work / dt / 1e12,
        "unit": "TFLOPS",
        "cores": threads,
        "nproc": host["nproc"],
        "cpu_model": host["cpu_model"],
        "omp_num_threads": host["omp_num_threads"],
        "kind": "port",
        "sample": (f"CPU oracle (C restatement of the reference CPU layer, OpenMP over heads) on the "
                   f"shifted 720p plan: video queries of {k} of {len(wins)} windows + text queries of "
                   f"every window, 20 heads; {work / 1e9:.1f} GFLOP in {dt:.1f} s"),
    }


def mapped_libraries(fragment: str) -> list:
    """Paths of the shared objects mapped into this process whose name holds
    `fragment` (which hipBLASLt copy the fp16 InnerProducts ran on)."""
    out = set()
    try:
        for line in Path("/proc/self/maps").read_text().splitlines():
            parts = line.split()
            if len(parts) >= 6 and fragment in parts[-1]:
                out.add(parts[-1])
    except OSError:
        pass
    return sorted(out)


def dit_step_cxx(steps: int) -> dict:
    """The same DiT forward driven from C++ through the C ABI alone
    (tests/cxx/dit_step, a child process without torch): the time a C++
    integration sees, on the libhipblaslt it maps itself (ROCm's), against
    dit_step's, whose process maps the copy bundled with torch."""
    exe = Path(__file__).resolve().parent / "tests" / "cxx" / "_build" / "dit_step"
    if not exe.exists():
        return {"error": "tests/cxx/_build/dit_step is not built (build() compiles it)"}
    try:
        proc = subprocess.run([str(exe), "--steps", str(steps), "--warmup", "1"], capture_output=True, text=True,
                              timeout=600)
    except subprocess.TimeoutExpired:
        return {"error": "dit_step timed out"}
    lines = [ln for ln in proc.stdout.splitlines() if ln.startswith("{")]
    if proc.returncode != 0 or not lines:
        return {"error": f"dit_step exited {proc.returncode}: {proc.stderr.strip()[-400:]}"}
    return json.loads(lines[-1])


def _median_ms(fn, runs=3):
    fn()  # warmup
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return float(np.median(ts))


def _gpu_ms(fn, reps=20):
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def _row(name, variant, ms, flops, nbytes):
    t = ms * 1e-3
    return {"config": name, "variant": variant, "gpu_ms": round(ms, 4), "tflops": round(flops / t / 1e12, 2),
            "mfma_pct": round(100 * flops / t / 1e12 / PEAK_FP16_TFLOPS, 2),
            "hbm_gbs": round(nbytes / t / 1e9, 1), "hbm_pct": round(100 * nbytes / t / 1e9 / PEAK_HBM_GBS, 2),
            "roofline_pct": round(100 * max(flops / (PEAK_FP16_TFLOPS * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)) / t, 2),
            "cpu_ms": None, "cpu_cores": None, "pass": None}


def config_table(dev):
    """The GPU side of one row per configuration of the metric's config list
    that fits a GPU and the CPU beside it: the single windowed MM-attention
    layer at the 480x256x5 grid 2x16x30 (config 1: fp32, no RoPE, no QK-norm,
    2x8x10 unshifted windows; config 2: fp16, QK-RMSNorm + RoPE, unshifted and
    shifted, and bf16 unshifted, whose P*V takes P as two bf16 terms) and one
    DiT block at that grid (config 4: hidden 2560, 20 heads,
    MLP 6912, fp16 weights N(0, 0.02^2), fp16 inputs N(0, 1), 58 text tokens).
    GPU ms: mean over 20 launches after 3 warmups (HIP events).  Config 3 is
    the line's own workload; config 5 the dit_step.

    Returns the rows and, per row, the host inputs and GPU outputs that the
    CPU-baseline leg (cpu_baseline_configs) times the oracle on and checks."""
    import torch
    import sv2hip
    from parity import cast_like, reference_freqs
    import ncnn_files as nf
    Tg, Hg, Wg, D = 2, 16, 30, HEADS * HD
    Lv = Tg * Hg * Wg
    freqs = reference_freqs()
    rows, cases = [], []
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    for name, in_dt, norm, rope, shifted in (("1", "f32", False, sv2hip.ROPE_NONE, False),
                                             ("2", "f16", True, sv2hip.ROPE_REFERENCE, False),
                                             ("2", "f16", True, sv2hip.ROPE_REFERENCE, True),
                                             ("2", "bf16", True, sv2hip.ROPE_REFERENCE, False)):
        rng = np.random.default_rng(31 + shifted)
        vid = cast_like(rng.standard_normal((Lv, 3 * D), dtype=np.float32), in_dt)
        txt = cast_like(rng.standard_normal((L_TXT, 3 * D), dtype=np.float32), in_dt)
        gam = list(rng.uniform(0.5, 1.5, (4, 128)).astype(np.float32)) if norm else None
        wins = sv2hip.window_plan(sv2hip.rule(Tg, Hg, Wg, shifted, 2, 8, 10))
        sizes = [(w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) for w in wins]
        flops = sum(4.0 * (v + L_TXT) ** 2 * HD * HEADS for v in sizes)
        es = 4 if in_dt == "f32" else 2
        nbytes = (Lv + L_TXT) * HEADS * HD * es * 4
        attn = sv2hip.WindowAttention(sv2hip.rule(Tg, Hg, Wg, shifted, 2, 8, 10), HEADS, L_TXT, qk_norm=norm,
                                      rope_mode=rope, freqs=freqs, device=dev)
        tv = torch.from_numpy(vid).to(dev, tdt[in_dt])
        tt = torch.from_numpy(txt).to(dev, tdt[in_dt])
        tg = None if gam is None else [torch.from_numpy(g).to(dev) for g in gam]
        ov = torch.empty((Lv, D), dtype=tdt[in_dt], device=dev)
        ot = torch.empty((L_TXT, D), dtype=tdt[in_dt], device=dev)
        ms = _gpu_ms(lambda: attn(tv, tt, tg, ov, ot))
        rows.append(_row(name, f"2x8x10 {'shifted' if shifted else 'unshifted'}, "
                               f"{'no RoPE / no QK-norm' if not norm else 'QK-RMSNorm + reference RoPE'}, {in_dt}",
                         ms, flops, nbytes))
        cases.append(dict(kind="attention", gpu=ov.float().cpu().numpy(), vid=vid, txt=txt, grid=(Tg, Hg, Wg),
                          in_dt=in_dt, norm=norm, rope=rope, freqs=freqs, gammas=gam, shifted=shifted))

    # config 4: one block, fp16 compute
    rng = np.random.default_rng(41)
    w = nf.random_weights(rng, D, DIT_FFN, shared=False)
    vid = rng.standard_normal((Lv, D), dtype=np.float32).astype(np.float16).astype(np.float32)
    txt = rng.standard_normal((L_TXT, D), dtype=np.float32).astype(np.float16).astype(np.float32)
    emb = rng.standard_normal(6 * D, dtype=np.float32)
    blk = sv2hip.DitBlock.from_host(sv2hip.block_config(dim=D, heads=HEADS, mlp_hidden=DIT_FFN, window_t=2,
                                                        window_h=8, window_w=10), w, sv2hip.F16)
    blk.set_runtime_shape(Tg, Hg, Wg)
    tv = torch.from_numpy(vid).to(dev, torch.float16)
    tt = torch.from_numpy(txt).to(dev, torch.float16)
    te = torch.from_numpy(emb).to(dev)
    ov, ot = torch.empty_like(tv), torch.empty_like(tt)
    ws = torch.empty(blk.workspace_size(L_TXT), dtype=torch.uint8, device=dev)
    ms = _gpu_ms(lambda: blk.forward(tv, tt, te, ov, ot, workspace=ws))
    gv = ov.float().cpu().numpy()
    blk.close()
    gemm = 2.0 * (Lv + L_TXT) * D * (3 * D + D + 3 * DIT_FFN)
    attn_f = sum(4.0 * (v + L_TXT) ** 2 * HD * HEADS for v in
                 [(x[1] - x[0]) * (x[3] - x[2]) * (x[5] - x[4])
                  for x in sv2hip.window_plan(sv2hip.rule(Tg, Hg, Wg, False, 2, 8, 10))])
    wbytes = 2 * 2 * (3 * D * D + D * D + 3 * D * DIT_FFN)  # two branches of fp16 matrices
    rows.append(_row("4", "one block 960+58 tokens, 2x8x10 unshifted, fp16 (video InnerProducts on hipBLASLt, "
                     "text rows on the few-row kernel)",
                     ms, gemm + attn_f, wbytes))
    cases.append(dict(kind="block", gpu=gv, weights=w, vid=vid, txt=txt, emb=emb, grid=(Tg, Hg, Wg)))
    return rows, cases


def cpu_baseline_configs(rows, cases):
    """The CPU-baseline leg of the per-configuration rows: the oracle's median
    of 3 after a warmup on each row's inputs, on the host cores, and the
    errors of the row's GPU outputs against the oracle's (the attention's
    gates: max-abs <= 2e-3 / mean-abs <= 2e-4 but for one-ulp bf16 flips; the
    block's, fp16 against the oracle's fp32 block: NRMSE <= 2e-3)."""
    import oracle
    from parity import cast_like, report
    oracle.load()
    host = host_cpu()
    threads = host["nproc"]
    if host["omp_num_threads"]:
        threads = min(threads, int(host["omp_num_threads"]))
    for row, c in zip(rows, cases):
        T_, H_, W_ = c["grid"]
        ref = {}
        if c["kind"] == "attention":
            def run():
                ref["v"], ref["t"] = oracle.window_attention(
                    c["vid"], c["txt"], T_, H_, W_, heads=HEADS, qk_norm=c["norm"], rope_mode=c["rope"],
                    freqs=c["freqs"], gammas=c["gammas"], shifted=c["shifted"], wt=2, wh=8, ww=10, threads=threads)
            cpu_ms = _median_ms(run)
            rep = report(c["gpu"], cast_like(ref["v"], c["in_dt"]))
            err = {"max_abs": rep["max_abs"], "mean_abs": rep["mean_abs"], "flips": rep["flips"]}
            passed = bool(rep["finite"] and rep["over_tol_not_flip"] == 0 and rep["mean_abs"] <= 2e-4)
        else:
            D = HEADS * HD

            def run():
                ref["v"], ref["t"] = oracle.block_forward(c["weights"], c["vid"], c["txt"], c["emb"], T_, H_, W_,
                                                          dim=D, heads=HEADS, mlp_hidden=DIT_FFN, shared=False,
                                                          shifted=False, wt=2, wh=8, ww=10, threads=threads)
            cpu_ms = _median_ms(run)
            d = c["gpu"].astype(np.float64) - ref["v"]
            rms = max(float(np.sqrt(np.mean(ref["v"].astype(np.float64) ** 2))), 1e-12)
            nrmse = float(np.sqrt(np.mean(d * d))) / rms
            err = {"max_abs": float(np.abs(d).max()), "mean_abs": float(np.abs(d).mean()), "nrmse": nrmse}
            passed = bool(np.isfinite(c["gpu"]).all() and nrmse <= 2e-3)
        row.update({"cpu_ms": round(cpu_ms, 1), "cpu_cores": threads, **err, "pass": passed})


DIT_DIM, DIT_FFN, DIT_BLOCKS, LATENT_C, TEXT_C, OUT_C = 2560, 6912, 32, 33, 5120, 16


def dit_flops():
    """Algorithmic flops of one DiT forward at 720p x 21f: every InnerProduct
    (2 * rows * in * out) plus the windowed attention of the 16 unshifted and
    16 shifted blocks (sum_w 4 * S_w^2 * 128 * 20)."""
    Lv, D, F = T * H * W, DIT_DIM, DIT_FFN
    gemm_block = 2.0 * (Lv + L_TXT) * D * (3 * D + D + 3 * F)
    heads = 2.0 * Lv * 4 * LATENT_C * D + 2.0 * L_TXT * TEXT_C * D + 2.0 * Lv * D * 4 * OUT_C
    attn = (DIT_BLOCKS // 2) * (plan_stats(False)[2] + plan_stats(True)[2])
    return DIT_BLOCKS * gemm_block + heads, attn


def dit_bench(dev, steps: int, warmup: int):
    """The full 32-block DiT forward of one Euler step at 1280x720x21: latent
    [33, 6, 90, 160] (16 noise + 16 condition channels N(0, 1), one channel of
    ones), 58 text tokens of width 5120 N(0, 1), timestep 1000; fp16 weights
    N(0, 0.02^2) generated on the device (q/k norm weights U(0.5, 1.5)),
    resident in HBM; blocks alternate unshifted / shifted 2x9x16 windows as
    the exporter lays them out (shared weights from block 10, the last block
    with the last-layer text rule)."""
    import torch
    import sv2hip
    from ncnn_files import MATRICES, block_flags, shapes
    from parity import reference_freqs

    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    D = DIT_DIM

    def randn(shape, dtype, std=0.02):
        return (torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std).to(dtype).contiguous()

    wbytes = [0]

    def branch():
        out = {}
        for f, shp in shapes(D, DIT_FFN).items():
            if f in ("norm_q", "norm_k"):
                out[f] = (torch.rand(shp, generator=g, device=dev) + 0.5).contiguous()
            else:
                out[f] = randn(shp, torch.float16 if f in MATRICES else torch.float32)
            wbytes[0] += out[f].numel() * out[f].element_size()
        return out

    weights, cfgs = [], []
    for i in range(DIT_BLOCKS):
        shared, last, shifted = block_flags(i, DIT_BLOCKS)
        w = {"vid": branch(), "freqs": reference_freqs()}
        if not shared:
            w["txt"] = branch()
        weights.append(w)
        cfgs.append(dict(block_index=i, shared_weights=int(shared), last_layer=int(last), shifted_window=int(shifted),
                         window_t=WIN[0], window_h=WIN[1], window_w=WIN[2]))
    f16, f32 = torch.float16, torch.float32
    wi = {"w_vid": randn((D, 4 * LATENT_C), f16), "b_vid": randn((D,), f32),
          "w_txt": randn((D, TEXT_C), f16), "b_txt": randn((D,), f32),
          "w_time_in": randn((D, 256), f32), "b_time_in": randn((D,), f32),
          "w_time_hid": randn((D, D), f32), "b_time_hid": randn((D,), f32),
          "w_time_out": randn((6 * D, D), f32), "b_time_out": randn((6 * D,), f32)}
    wo = {"norm_weight": (torch.rand((D,), generator=g, device=dev) + 0.5).contiguous(),
          "shift": randn((D,), f32), "scale": randn((D,), f32),
          "w_proj": randn((4 * OUT_C, D), f16), "b_proj": randn((4 * OUT_C,), f32)}
    inp = sv2hip.DitInput.create(wi, sv2hip.F16, on_device=True)
    outp = sv2hip.DitOutput.create(wo, sv2hip.F16, on_device=True)
    latent = torch.randn((LATENT_C, T, 2 * H, 2 * W), generator=g, device=dev)
    latent[LATENT_C - 1].fill_(1.0)
    text = torch.randn((L_TXT, TEXT_C), generator=g, device=dev)
    out = torch.empty((OUT_C, T, 2 * H, 2 * W), device=dev)
    stream = torch.cuda.current_stream()

    def timed(fused: bool):
        # the blocks borrow the same device weights; fused selects the
        # hand-written MFMA InnerProducts with their passes fused in
        blocks = [sv2hip.DitBlock.from_device(sv2hip.block_config(fused_gemm=int(fused), **c), w, sv2hip.F16)
                  for c, w in zip(cfgs, weights)]
        dit = sv2hip.Dit.create(inp, blocks, outp)
        ws = torch.empty(dit.workspace_size(T, 2 * H, 2 * W, L_TXT), dtype=torch.uint8, device=dev)
        for _ in range(warmup):
            dit.forward(latent, text, 1000.0, out, workspace=ws, stream=stream)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in ev:
            a.record(stream)
            dit.forward(latent, text, 1000.0, out, workspace=ws, stream=stream)
            b.record(stream)
        torch.cuda.synchronize()
        t = float(np.mean([a.elapsed_time(b) for a, b in ev]))
        ok = bool(torch.isfinite(out).all().item())
        dit.close()
        for blk in blocks:
            blk.close()
        del ws
        return t, ok

    ms, finite = timed(False)
    ms_fused, finite_fused = timed(True)
    gemm_f, attn_f = dit_flops()
    return {
        "ms": round(ms, 3),
        "steps": steps,
        "tflop": round((gemm_f + attn_f) / 1e12, 2),
        "tflops": round((gemm_f + attn_f) / (ms * 1e-3) / 1e12, 1),
        "mfma_util": round((gemm_f + attn_f) / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
        "gemm_tflop": round(gemm_f / 1e12, 2),
        "attention_tflop": round(attn_f / 1e12, 2),
        "block_weights_gb": round(wbytes[0] / 1e9, 2),
        "output_finite": finite,
        "fused_inner_products_ms": round(ms_fused, 3),
        "fused_inner_products_finite": finite_fused,
        "workload": ("SeedVR2-3B DiT forward, 1280x720x21 (latent 33x6x90x160 -> grid 6x45x80), 32 blocks, "
                     "hidden 2560, 20 heads, MLP 6912 SwiGLU, 58 text tokens, windows 2x9x16 alternating "
                     "unshifted / shifted, fp16 weights and activations, fp32 accumulation"),
    }


def elementwise_bench(dev, reps: int = 20):
    """The block's row-wise kernels at the 720p x 21f DiT shape (21600 video +
    58 text rows, merged as in the shared-weight blocks; hidden 2560, MLP
    6912; fp16 rows, fp32 modulation vectors): per kernel the mean device time
    of `reps` launches captured in one HIP graph and its algorithmic HBM bytes
    (each element read and written once: RMSNorm + ada 2 + 2 B, the gated
    residual in place 2 + 2 + 2 B, SwiGLU in place 2 + 2 + 2 B).  The in-place
    kernels run on values kept bounded (|gate| < 1, value in [0.5, 1))."""
    import torch
    import sv2hip

    g = torch.Generator(device=dev)
    g.manual_seed(7)
    rows, D, F = T * H * W + L_TXT, DIT_DIM, DIT_FFN
    f16 = torch.float16
    x = torch.randn((rows, D), generator=g, device=dev).to(f16)
    y = torch.empty_like(x)
    res = torch.randn((rows, D), generator=g, device=dev).to(f16)
    emb = torch.randn(6 * D, generator=g, device=dev) * 0.02
    shift = torch.randn(D, generator=g, device=dev) * 0.02
    scale = torch.randn(D, generator=g, device=dev) * 0.02
    gate_vec = torch.rand(D, generator=g, device=dev) * 0.5
    hx = torch.randn((rows, F), generator=g, device=dev).to(f16)
    hv = (torch.rand((rows, F), generator=g, device=dev) * 0.5 + 0.5).to(f16)
    cur = torch.cuda.current_stream
    ops = {
        "rmsnorm_ada": (lambda: sv2hip.rmsnorm_ada(x, y, 1e-5, emb, shift, scale, 0, True, stream=cur()),
                        rows * D * 4),
        "ada_residual": (lambda: sv2hip.ada_residual(y, res, emb, gate_vec, 0, 0, stream=cur()), rows * D * 6),
        "swiglu": (lambda: sv2hip.swiglu(hx, hv, stream=cur()), rows * F * 6),
    }
    out = {}
    for name, (fn, nbytes) in ops.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(cur())
        graph.replay()
        b.record(cur())
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        out[name] = {"us": round(us, 2), "bytes": nbytes, "gbs": round(nbytes / us / 1e3, 1),
                     "hbm_util": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4)}
        del graph
    out["workload"] = ("row-wise kernels at 1280x720x21: 21658 rows x 2560 (RMSNorm + ada, gated residual) and "
                       "21658 x 6912 (SwiGLU), fp16")
    return out


def text_products_bench(dev):
    """The text branch's four InnerProducts at 58 rows (the DiT's text tokens;
    hidden 2560, MLP 6912, fp16): the few-row kernel with its pass fused
    (sv2_inner_product_f16_few) against torch.matmul (hipBLASLt) plus the
    separate pass the library path runs after it (proj: the gated residual;
    gate/in: SwiGLU; the out product's gated residual rides in the library's
    epilogue, so its library figure is the product alone).  Weights are
    rotated over copies of at least 700 MB so every launch streams its weight
    matrix from HBM, as each block's does in a forward; mean device time of
    3 launches per copy, replayed from a HIP graph."""
    import math
    import torch
    import sv2hip

    g = torch.Generator(device=dev)
    g.manual_seed(58)
    M, D, F = L_TXT, DIT_DIM, DIT_FFN
    f16 = torch.float16
    cur = torch.cuda.current_stream
    emb = torch.randn(6 * D, generator=g, device=dev) * 0.02
    gate_vec = torch.rand(D, generator=g, device=dev) * 0.5
    bias = torch.randn(D, generator=g, device=dev) * 0.02
    lib = sv2hip.load()
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=dev)

    def timed(fn, reps):
        # captured in one HIP graph, so host launch overhead does not enter
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(reps):
                fn(i)
        graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(cur())
        graph.replay()
        b.record(cur())
        torch.cuda.synchronize()
        del graph
        return a.elapsed_time(b) * 1e3 / reps

    out = {}
    for name, K, N, epi in (("qkv", D, 3 * D, sv2hip.EPI_STORE), ("proj", D, D, sv2hip.EPI_RESIDUAL),
                            ("gate_in", D, F, sv2hip.EPI_SWIGLU), ("out", F, D, sv2hip.EPI_RESIDUAL)):
        nw = 2 if epi == sv2hip.EPI_SWIGLU else 1
        wbytes = N * K * 2 * nw
        R = max(4, math.ceil(700e6 / wbytes))
        x = torch.randn((M, K), generator=g, device=dev).to(f16)
        w1 = [(torch.randn((N, K), generator=g, device=dev) * 0.02).to(f16) for _ in range(R)]
        w2 = [(torch.randn((N, K), generator=g, device=dev) * 0.02).to(f16) for _ in range(R)] if nw == 2 else None
        res = torch.randn((M, N), generator=g, device=dev).to(f16)
        y = torch.empty((M, N), dtype=f16, device=dev)
        y2 = torch.empty_like(y)
        gt = gate_vec[:N] if N == D else None
        bs = bias if name == "proj" else None

        def few(i):
            sv2hip.inner_product_f16_few(x, w1[i % R], y, epi, w_value=w2[i % R] if w2 else None,
                                         bias=bs, gate=gt if epi == sv2hip.EPI_RESIDUAL else None,
                                         residual=res if epi == sv2hip.EPI_RESIDUAL else None, workspace=ws,
                                         stream=cur())

        def library(i):
            torch.matmul(x, w1[i % R].t(), out=y)
            if name == "proj":
                sv2hip.ada_residual(y, res, emb, gate_vec, 0, 0, stream=cur())
            elif name == "gate_in":
                torch.matmul(x, w2[i % R].t(), out=y2)
                sv2hip.swiglu(y, y2, stream=cur())

        t_few = timed(few, 3 * R)
        t_lib = timed(library, 3 * R)
        out[name] = {"in": K, "out": N, "weight_mb": round(wbytes / 1e6, 1), "few_us": round(t_few, 2),
                     "library_us": round(t_lib, 2), "few_gbs": round(wbytes / t_few / 1e3, 1),
                     "splits": int(max(1, lib.sv2_inner_product_f16_few_workspace(M, K, N, epi)
                                       // max(1, M * N * 4)))}
        del w1, w2
        torch.cuda.empty_cache()
    out["workload"] = ("text-branch InnerProducts at 58 rows (2560 -> 7680; 2560 -> 2560 + gated residual; "
                       "2560 -> 2 x 6912 + SwiGLU; 6912 -> 2560 + gated residual), fp16, weights from HBM")
    return out


def sampler_bench(dev, reps: int = 50):
    """The sampler half of one Euler step at 1280x720x21 (latent 16x6x90x160,
    fp32, resident): the 33-channel DiT input, CFG 6.5 with rescale 0.7 of two
    predictions, and the Euler update; per operation the mean time over
    `reps` launches and its algorithmic HBM bytes (each element read and
    written once per pass: DiT input 65 x 4 B per token, CFG 12 B + the
    rescale pass 8 B per element, Euler 12 B per element).

    The `reps` launches of an operation are captured in one HIP graph and
    the replay is timed, so "us" is the device time of its kernels; an eager
    loop of these few-microsecond launches measures the host's launch rate
    instead, reported as "us_eager"."""
    import torch
    import sv2hip

    g = torch.Generator(device=dev)
    g.manual_seed(99)
    shape = (16, T, 2 * H, 2 * W)
    n = 16 * T * 4 * H * W
    lat, cond, pos, neg = (torch.randn(shape, generator=g, device=dev) for _ in range(4))
    s = sv2hip.EulerSampler(50)
    dit_in = torch.empty((33,) + shape[1:], device=dev)
    guided = torch.empty_like(lat)
    nxt = torch.empty_like(lat)
    cur = torch.cuda.current_stream  # the capture stream inside a graph capture
    ops = {
        "dit_input": (lambda: s.make_dit_input(lat, cond, output=dit_in, stream=cur()), 65 * 4 * n // 16),
        "cfg_rescale": (lambda: s.apply_cfg(pos, neg, 6.5, 0.7, output=guided, stream=cur()), 20 * n),
        "euler_step": (lambda: s.step_to(guided, lat, 980.0, 960.0, output=nxt, stream=cur()), 12 * n),
    }
    out = {}
    for name, (fn, nbytes) in ops.items():
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(cur())
        for _ in range(reps):
            fn()
        b.record(cur())
        torch.cuda.synchronize()
        us_eager = a.elapsed_time(b) * 1e3 / reps
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        a.record(cur())
        graph.replay()
        b.record(cur())
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        del graph
        out[name] = {"us": round(us, 2), "us_eager": round(us_eager, 2), "bytes": nbytes,
                     "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "hbm_util": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    out["step_us"] = round(sum(v["us"] for v in out.values()), 2)
    out["workload"] = "sampler step at 1280x720x21: latent 16x6x90x160 fp32, CFG 6.5 rescale 0.7, Euler 980->960"
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    ap.add_argument("--no-table", action="store_true",
                    help="skip the per-configuration rows (configs 1, 2 and 4 on the GPU and the CPU oracle)")
    ap.add_argument("--dit-steps", type=int, default=3, help="timed DiT forwards (0 skips the DiT leg)")
    ap.add_argument("--dit-only", action="store_true",
                    help="run only the DiT leg and print its figures (for profiling the DiT step)")
    ap.add_argument("--elementwise-only", action="store_true",
                    help="run only the row-wise kernels' leg and print its figures (for profiling them)")
    ap.add_argument("--text-products-only", action="store_true",
                    help="run only the text-branch InnerProducts' leg and print its figures")
    ap.add_argument("--sampler-only", action="store_true",
                    help="run only the sampler leg and print its figures (for profiling the sampler kernels)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only copy a device buffer of BYTES three times (a plain copy kernel of known "
                         "size, to calibrate the FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)

    import torch
    import sv2hip
    from parity import reference_freqs

    dev = torch.device("cuda:0")
    if args.copy_probe:
        src = torch.ones(args.copy_probe // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4}))
        return
    sv2hip.load()
    if args.elementwise_only:
        print(json.dumps({"elementwise": elementwise_bench(dev)}))
        return
    if args.sampler_only:
        print(json.dumps({"sampler_step": sampler_bench(dev)}))
        return
    if args.text_products_only:
        print(json.dumps({"text_products": text_products_bench(dev)}))
        return
    if args.dit_only:
        print(json.dumps({"dit_step": dit_bench(dev, max(args.dit_steps, 1), 1)}))
        return
    D = HEADS * HD
    rng = np.random.default_rng(0)
    vid = torch.from_numpy(rng.standard_normal((T * H * W, 3 * D), dtype=np.float32)).to(dev, torch.float16)
    txt = torch.from_numpy(rng.standard_normal((L_TXT, 3 * D), dtype=np.float32)).to(dev, torch.float16)
    gam = [torch.from_numpy(g).to(dev) for g in rng.uniform(0.5, 1.5, (4, 128)).astype(np.float32)]
    freqs = reference_freqs()
    layers = []
    for shifted in (False, True):
        attn = sv2hip.WindowAttention(sv2hip.rule(T, H, W, shifted, *WIN), HEADS, L_TXT, freqs=freqs,
                                      device=dev)
        _, _, flops = plan_stats(shifted)
        layers.append((shifted, attn, flops))
    out_v = torch.empty((T * H * W, D), dtype=torch.float16, device=dev)
    out_t = torch.empty((L_TXT, D), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream()

    def step(events=None):
        for i, (_, attn, _) in enumerate(layers):
            if events is not None:
                events[i][0].record(stream)
            attn(vid, txt, gam, out_v, out_t, stream=stream)
            if events is not None:
                events[i][1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in layers] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(ev[k])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_layer_ms = [float(np.mean([ev[k][i][0].elapsed_time(ev[k][i][1]) for k in range(args.steps)]))
                    for i in range(len(layers))]
    flops_step = sum(f for _, _, f in layers)
    ms_step = wall * 1e3 / args.steps
    tflops = flops_step / (ms_step * 1e-3) / 1e12
    B = algorithmic_bytes()
    variants = {}
    for (shifted, _, flops), ms in zip(layers, per_layer_ms):
        t = ms * 1e-3
        variants["shifted" if shifted else "unshifted"] = {
            "ms": round(ms, 4),
            "tflops": round(flops / t / 1e12, 2),
            "mfma_util": round(flops / t / 1e12 / PEAK_FP16_TFLOPS, 4),
            "hbm_gbs": round(B / t / 1e9, 1),
            "hbm_util": round(B / t / 1e9 / PEAK_HBM_GBS, 4),
            "roofline_frac": round(max(flops / (PEAK_FP16_TFLOPS * 1e12), B / (PEAK_HBM_GBS * 1e9)) / t, 4),
        }
    # the window kernel alone (its text inputs prepared once, then only the
    # SV2_ATTN_STAGE_WINDOWS launch repeated): the dominant kernel's own
    # launch time for the roofline, comparable with a kernel trace
    kernel_ms = []
    for (shifted, attn, _) in layers:
        attn(vid, txt, gam, out_v, out_t, stream=stream, stages=sv2hip.STAGE_TEXT_PREPARE)
        for _ in range(3):
            attn(vid, txt, gam, out_v, out_t, stream=stream, stages=sv2hip.STAGE_WINDOWS)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(args.steps):
            attn(vid, txt, gam, out_v, out_t, stream=stream, stages=sv2hip.STAGE_WINDOWS)
        b.record(stream)
        torch.cuda.synchronize()
        kernel_ms.append(a.elapsed_time(b) / args.steps)
        variants["shifted" if shifted else "unshifted"]["kernel_ms"] = round(kernel_ms[-1], 4)
        variants["shifted" if shifted else "unshifted"]["kernel_tflops"] = round(
            layers[int(shifted)][2] / (kernel_ms[-1] * 1e-3) / 1e12, 2)
    t_launch = float(np.mean(kernel_ms)) * 1e-3
    achieved = B / t_launch / 1e9
    traffic, traffic_source = measured_traffic()

    result = {
        "metric": "window-attn TFLOPS & % fp16 MFMA peak; DiT step ms @720p×21f, 1 GPU",
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": ("windowed MM-attention 720p x 21f: grid 6x45x80 (21600 video tokens), windows "
                         "2x9x16, step = unshifted layer (75 windows) + shifted layer (144 ragged windows), "
                         "20 heads x 128, 58 joint text tokens, fp16 N(0,1) q/k/v, QK-RMSNorm + RoPE "
                         "(reference mmrope3d)"),
            "mfma": "bf16 QK^T (exact bf16 q/k), f16 PV, f32 accumulate",
            "mfma_util": round(tflops / PEAK_FP16_TFLOPS, 4),
            "variants": variants,
            "dit_step_ms": None,
            "dit_step": None,
            "sampler_step": None,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel": "window_attention_kernel<F16, reference RoPE> alone (sv2_window_attention_stages, "
                      "SV2_ATTN_STAGE_WINDOWS), mean launch time of the two variants with HIP events on the launch "
                      "stream; variants[].ms are whole layers (text prologue + window kernel + text reduction)",
        },
    }
    if args.dit_steps > 0:
        ds = dit_bench(dev, args.dit_steps, 1)
        result["config"]["dit_step_ms"] = ds["ms"]
        result["config"]["dit_step"] = ds
        result["config"]["dit_step_cxx"] = dit_step_cxx(args.dit_steps)
    result["config"]["sampler_step"] = sampler_bench(dev)
    result["config"]["elementwise"] = elementwise_bench(dev)
    result["config"]["text_products"] = text_products_bench(dev)
    table = config_table(dev) if not args.no_table else None
    if table is not None:
        result["config"]["configs"] = table[0]
    result["config"]["hipblaslt_mapped"] = mapped_libraries("libhipblaslt")
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
        if table is not None:
            cpu_baseline_configs(*table)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
