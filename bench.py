"""Benchmark of the crbq hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--method crb]

Workload (per layer; metric quoted on OPT-6.7B
shapes): one OPT-6.7B-shaped decoder layer, random-init fp16 weights
W ~ N(0, 0.02^2) for k/v/q/out_proj 4096x4096, fc1 16384x4096 and
fc2 4096x16384, with 128 x 2048 synthetic fp16 calibration tokens per
distinct sublayer input (Gaussian with heavy-tailed Student-t(4) channel
scales; there is no network for checkpoints or datasets).  One step =
Hessian accumulation of all 4 distinct inputs + damped inverse factor +
the full CRB block loop (blocksize 128, hessian salient metric) of all 6
sublayers, with every input already resident in HBM.  A 32-layer stack
runs 32 such steps (plus the decoder forwards, which are not timed here).

Prints one JSON line: value = seconds per layer (lower is better), with
cols/s, phase split, the roofline of the dominant kernel (Hessian SYRK on
bf16/f16 MFMA), and the CPU baseline (the test-only oracle on this host's
cores, on a bounded sample, extrapolated to one layer).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from crb_amd import synth  # noqa: E402

METRIC = "CRB quantize time/layer (s) + cols/s, OPT-6.7B shapes; MFMA util & HBM GB/s"
PEAK_F16 = 2.5e15       # dense f16/bf16 MFMA, MI355X
PEAK_F32 = 157.3e12     # fp32 MFMA
PEAK_HBM = 8.0e12


def make_layer(dev, seed=0):
    subs = synth.opt_sublayers("opt-6.7b")
    Ws = {}
    for i, (name, r, c, grp) in enumerate(subs):
        g = torch.Generator(device=dev)
        g.manual_seed(seed * 100 + i)
        Ws[name] = (torch.randn(r, c, generator=g, device=dev) * 0.02).half()
    return subs, Ws


def make_inputs(dev, ntok, seed=0, fc2_first=True):
    """One [ntok, C] fp16 activation per distinct sublayer input, in the
    order their Hessians are accumulated.  With fc2_first the fc2 input
    (C = 16384), whose Hessian, factor and block loop form the layer's
    longest chain, comes first and the other inputs' work overlaps it."""
    shapes = {"qkv": 4096, "out": 4096, "fc1": 4096, "fc2": 16384}
    if fc2_first:
        shapes = {"fc2": 16384, **{k: v for k, v in shapes.items() if k != "fc2"}}
    X = {}
    for j, (grp, C) in enumerate(shapes.items()):
        s = synth.channel_scales(C, seed + j, kind="student_t4", device=dev)
        g = torch.Generator(device=dev)
        g.manual_seed(seed * 1000 + j)
        x = torch.empty(ntok, C, dtype=torch.float16, device=dev)
        step = 8192
        for t0 in range(0, ntok, step):
            t1 = min(ntok, t0 + step)
            x[t0:t1] = (torch.randn(t1 - t0, C, generator=g, device=dev) * s).half()
        X[grp] = x
    return X


def one_layer(subs, W0, X, method, timing):
    """One step.  The driver brackets every Hessian launch with HIP events on
    the stream it runs on (LayerQuantizer.syrk_ms)."""
    from crb_amd.driver import LayerQuantizer, PhaseTimes, Sublayer
    sl = [Sublayer(n, W0[n].clone(), g) for (n, r, c, g) in subs]
    lq = LayerQuantizer(sl, method=method)
    pt = PhaseTimes() if timing else None
    for grp, x in X.items():
        lq.add_batch(grp, x)
    lq.quantize(pt)
    return lq, pt


def load_traffic(name):
    """HBM bytes per launch of the dominant kernel, measured by rocprofv3
    (FETCH_SIZE + WRITE_SIZE, calibrated on a copy kernel) and recorded in
    profiles/; None if no such measurement is recorded."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                vals["t"] = float(line.split(":", 1)[1])
    return vals.get("t")


def load_profile_values(name):
    """`key: value` lines of a summary in profiles/ (None if it is absent)."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            k, sep, v = line.partition(":")
            if sep and k.strip().replace("_", "").isalnum() and " " not in k.strip():
                try:
                    vals[k.strip()] = float(v)
                except ValueError:
                    pass
    return vals


def stack_run(dev, nlayers, ntok, chunk=8, seed=0):
    """The model-level driver (crb_amd/stack.py) on an OPT-6.7B-shaped decoder
    stack of nlayers random-init layers, calibration 128 x 2048 uniform token
    ids: per layer the hooked capture forward, the quantization and the
    forward with the quantized weights.  Layer 0 (first use of the forward
    kernels) is not averaged."""
    from transformers import OPTConfig, OPTForCausalLM
    from crb_amd.stack import StackQuantizer
    torch.manual_seed(seed)
    cfg = OPTConfig(hidden_size=4096, ffn_dim=16384, num_attention_heads=32,
                    num_hidden_layers=nlayers, max_position_embeddings=2048, vocab_size=50272,
                    word_embed_proj_dim=4096, torch_dtype=torch.float16)
    with torch.device(dev):
        model = OPTForCausalLM(cfg).half().eval()
    seq = 2048
    g = torch.Generator().manual_seed(seed + 1)
    samples = torch.randint(0, cfg.vocab_size, (ntok // seq, seq), generator=g).to(dev)
    sq = StackQuantizer(model, chunk=chunk)
    t0 = time.time()
    stats = sq.run(samples)
    torch.cuda.synchronize()
    wall = time.time() - t0
    used = stats[1:] if len(stats) > 1 else stats
    mean = lambda f: sum(f(s) for s in used) / len(used)
    cap, hs = mean(lambda s: s.capture_ms), mean(lambda s: s.hessian_ms)
    qz, fw = mean(lambda s: s.quantize_ms), mean(lambda s: s.forward_ms)
    return {"layers": nlayers, "layers_averaged": len(used), "chunk": chunk,
            "s_per_layer_with_capture": round((cap + hs + qz + fw) / 1e3, 4),
            "s_per_layer_quantize": round((hs + qz) / 1e3, 4),
            "capture_forward_ms": round(cap, 2), "hessian_ms": round(hs, 2),
            "factors_blocks_ms": round(qz, 2), "quantized_forward_ms": round(fw, 2),
            "wall_s_all_layers": round(wall, 2)}


def packed_gemv(dev, R=4096, C=16384, reps=20):
    """Packed 3-bit GEMV (crbq_gemv_packed, 1-16 tokens) and GEMM
    (crbq_gemm_packed, 64 and 256 tokens) on the fc2 shape against torch's
    dense fp16 product with the same weights, per launch, from captured HIP
    graphs of `reps` launches (host call overhead excluded).  Random packed
    data: the kernels' work does not depend on the values."""
    from crb_amd import kernels
    torch.manual_seed(0)
    nblk = C // 128
    codes = torch.randint(0, 256, (R, nblk * 32), dtype=torch.uint8, device=dev)
    lut = torch.sort(torch.randn(R, nblk, 8, device=dev) * 0.02, dim=-1)[0].half()
    sal = torch.randint(0, 256, (nblk, 16), dtype=torch.uint8, device=dev)
    W = kernels.unpack(codes, lut, sal, C)
    nbytes = codes.numel() + lut.numel() * 2 + sal.numel()

    def graph_us(fn):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(5):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / (5 * reps)

    out = {"shape": [R, C], "dtype": "f16", "packed_bytes": nbytes,
           "bits_per_weight": round(nbytes * 8 / (R * C), 3), "per_nvec": {}}
    for nvec in (1, 8, 16):
        x = torch.randn(nvec, C, device=dev).half()
        tp = graph_us(lambda: kernels.gemv_packed(codes, lut, sal, C, x))
        td = graph_us(lambda: torch.nn.functional.linear(x, W))
        out["per_nvec"][nvec] = {"packed_us": round(tp, 2), "dense_fp16_us": round(td, 2),
                                 "packed_weight_GB_s": round(nbytes / tp / 1e3, 1),
                                 "dense_weight_GB_s": round(R * C * 2 / td / 1e3, 1)}
    out["gemm_per_ntok"] = {}
    for ntok in (64, 256):
        x = torch.randn(ntok, C, device=dev).half()
        tp = graph_us(lambda: kernels.gemm_packed(codes, lut, sal, C, x))
        td = graph_us(lambda: torch.nn.functional.linear(x, W))
        out["gemm_per_ntok"][ntok] = {"packed_us": round(tp, 2), "dense_fp16_us": round(td, 2),
                                      "packed_TFLOP_s": round(2 * R * C * ntok / tp / 1e6, 1)}
    return out


def _ev_ms(fn, reps):
    """Average ms of fn() over reps back-to-back calls, events recorded on
    the current stream (the one the wrappers launch on)."""
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def _graph_ms(fn, reps, warm=4, rounds=5):
    """Average ms of one fn() launch: reps calls captured in a HIP graph;
    `warm` untimed replays (the kernel's own steady state, not the clock
    the previous measurement left), then the median of `rounds` replays,
    each between two events recorded on the replay stream."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            for _ in range(reps):
                fn()
    torch.cuda.synchronize()
    for _ in range(warm):
        gr.replay()
    torch.cuda.synchronize()
    ms = []
    for _ in range(rounds):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            a.record(s)
            gr.replay()
            b.record(s)
        torch.cuda.synchronize()
        ms.append(a.elapsed_time(b) / reps)
    return sorted(ms)[len(ms) // 2]


def binarize_rates(dev, reps=20, methods=(("crb", 2), ("crb", 1), ("braq", 2), ("crbog", 2)),
                   sustained=True):
    """k_binarize_g over 524288 rows x 128 columns per launch (604 MB: the
    launch gaps amortized), 9 bytes per element (fp32 in, mask byte, fp32
    out) against HBM: launches of crbq_binarize through the C ABI (uint8
    mask prepared once) captured in a HIP graph and replayed between two
    events on the replay stream, so the figure is the kernel's and not the
    Python wrapper's.  For crb order 2 also `sustained`: 40 times as many
    launches as one continuous stream (about 0.1 s)."""
    from crb_amd import _lib
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    nb = 524288
    x = torch.randn(nb, 128, device=dev, generator=g) * 0.02
    m = (torch.rand(nb, 128, device=dev, generator=g) < 0.9).to(torch.uint8)
    ob = torch.empty_like(x)
    lib = _lib.ready(dev)
    out = {}
    for method, order in methods:
        def launch(method=method, order=order):
            st = torch.cuda.current_stream().cuda_stream
            _lib.check(lib.crbq_binarize(x.data_ptr(), nb, 128, 128, m.data_ptr(), 128, order,
                                         _lib.METHODS[method], 1e-5, 0.1, 1, ob.data_ptr(),
                                         128, st), "crbq_binarize")
        ms = _graph_ms(launch, reps)
        by = nb * 128 * 9
        rec = {
            "kernel": "k_binarize_g (8 lanes x 16 columns per row)", "shape": [nb, 128],
            "ms": round(ms, 5), "achieved": round(by / ms / 1e6, 1), "peak": PEAK_HBM / 1e9,
            "unit": "GB/s", "frac": round(by / ms / 1e6 / (PEAK_HBM / 1e9), 3)}
        if sustained and method == "crb" and order == 2:
            ms_s = _graph_ms(launch, reps * 40, warm=1, rounds=1)
            rec["sustained"] = {"ms": round(ms_s, 5), "launches": reps * 40,
                                "frac": round(by / ms_s / 1e6 / (PEAK_HBM / 1e9), 3)}
        out[f"{method}_order{order}"] = rec
    del x, m, ob
    return out


def kernel_rooflines(dev, R=4096, C=16384, reps=20, binarize=None):
    """The block loop's kernels launched alone at the fc2 sublayer's shapes
    (R x C = 4096 x 16384, 128-column blocks, 1024-column super-blocks),
    each against its roofline:
    * trailing update W[:, sb1:] -= Err @ U[sb0:sb1, sb1:] (k_sgemm, fp32
      MFMA), K = 1024, N = 8192 remaining columns: 2 M N K flop;
    * binarization (binarize_rates; given when measured earlier, before the
      layer steps, and then crb order 2 measured again here);
    * one block step (salient/split search + binarize + in-block error
      feedback, crbq_fasterquant on a 4096 x 128 block): its algorithmic
      bytes (W block in, U block in, Q, Err and masks out) against HBM;
    * the whole fc2 block loop alone (128 blocks, with trailing updates),
      and fc1's (16384 x 4096, 32 blocks);
    * q/k/v/out_proj's four 4096 x 4096 loops one by one and batched."""
    from crb_amd import _lib, kernels
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    out = {}
    # trailing update
    K, N = 1024, 8192
    Wbig = torch.randn(R, C, device=dev, generator=g) * 0.02
    Ubig = torch.randn(K, C, device=dev, generator=g) * 0.01
    E = torch.randn(R, K, device=dev, generator=g) * 0.01
    ms = _ev_ms(lambda: kernels.sgemm(E, Ubig[:, C - N:], Wbig[:, C - N:], alpha=-1.0,
                                      beta=1.0), reps)
    fl = 2.0 * R * N * K
    out["trailing_update_gemm"] = {
        "kernel": "k_sgemm<128> (fp32 MFMA)", "shape": [R, N, K], "ms": round(ms, 4),
        "achieved": round(fl / ms / 1e9, 1), "peak": PEAK_F32 / 1e12, "unit": "TFLOP/s",
        "frac": round(fl / ms / 1e9 / (PEAK_F32 / 1e12), 3)}
    if binarize is None:
        out["binarize"] = binarize_rates(dev, reps)
    else:
        # measured before the layer steps; the headline one again now, on a
        # chip that has just run at its power limit for seconds
        out["binarize"] = binarize
        out["binarize_after_layer_steps"] = binarize_rates(dev, reps, (("crb", 2),),
                                                           sustained=False)
    # one block step and the whole loop
    p = _lib.params("crb")
    U = torch.triu(torch.randn(C, C, device=dev, generator=g) * 1e-3)
    U.diagonal().add_(1.0)
    L = torch.zeros(R, device=dev)
    Wb = torch.empty(R, 128, device=dev)
    W0b = Wbig[:, :128].contiguous()

    def step():
        Wb.copy_(W0b)
        kernels.fasterquant_blocks(Wb, U[:128, :128], p, L, want_masks=False)

    ms_copy = _ev_ms(lambda: Wb.copy_(W0b), reps)
    ms = _ev_ms(step, reps) - ms_copy
    by = R * 128 * 4 * 3 + 128 * 128 * 4 + R * 128
    out["block_step"] = {
        "kernels": "colscore, phase_a, qpass1, qlist, qselect, phase_c, quantize",
        "shape": [R, 128], "ms": round(ms, 4), "achieved": round(by / ms / 1e6, 1),
        "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": round(by / ms / 1e6 / (PEAK_HBM / 1e9), 4),
        "note": "2 MB working set per block, resident in L2/MALL; bound by the search's "
                "dependent passes, not by HBM"}
    del Ubig, E
    W = Wbig.clone()

    def loop():
        W.copy_(Wbig)
        kernels.fasterquant_blocks(W, U, p, L, want_masks=False)

    ms = _ev_ms(loop, 2)
    out["block_loop_fc2_alone_ms"] = round(ms, 3)
    del W, Wbig, U
    # fc1's shape: 16384 rows x 4096 columns, 32 blocks
    R1, C1 = 4 * R, C // 4
    W1 = torch.randn(R1, C1, device=dev, generator=g) * 0.02
    U1 = torch.triu(torch.randn(C1, C1, device=dev, generator=g) * 1e-3)
    U1.diagonal().add_(1.0)
    L1 = torch.zeros(R1, device=dev)
    Wq = W1.clone()

    def loop1():
        Wq.copy_(W1)
        kernels.fasterquant_blocks(Wq, U1, p, L1, want_masks=False)

    out["block_loop_fc1_alone_ms"] = round(_ev_ms(loop1, 2), 3)
    del W1, U1, Wq
    # q/k/v/out_proj's shape (four 4096 x 4096 sublayers, the first three
    # sharing one factor, out_proj with its own): four block loops one after
    # another against one batched loop (crbq_fasterquant_batched), as the
    # layer driver runs them
    C4 = C // 4
    W4 = [torch.randn(R, C4, device=dev, generator=g) * 0.02 for _ in range(4)]
    U4 = []
    for _ in range(2):
        u = torch.triu(torch.randn(C4, C4, device=dev, generator=g) * 1e-3)
        u.diagonal().add_(1.0)
        U4.append(u)
    U4 = [U4[0], U4[0], U4[0], U4[1]]
    L4 = [torch.zeros(R, device=dev) for _ in range(4)]
    Wc = [w.clone() for w in W4]

    def loops_one_by_one():
        for w, w0, u, l in zip(Wc, W4, U4, L4):
            w.copy_(w0)
            kernels.fasterquant_blocks(w, u, p, l, want_masks=False)

    def loop_batched():
        for w, w0 in zip(Wc, W4):
            w.copy_(w0)
        kernels.fasterquant_blocks_batched(Wc, U4, p, L4)

    out["block_loops_qkvo_alone_ms"] = {"one_by_one": round(_ev_ms(loops_one_by_one, 2), 3),
                                        "batched": round(_ev_ms(loop_batched, 2), 3)}
    del W4, U4, L4, Wc
    torch.cuda.empty_cache()
    # inverse factor alone (crbq_hinv_upper: damping, Cholesky-inverse of the
    # index-reversed H, U) on a well-conditioned H of the fc2 input's size and
    # of the other inputs'; 2C^3/3 flop against the fp32 MFMA peak.  H is
    # refreshed before each call (the call damps it in place); that copy is
    # timed on its own and subtracted.  The calls are enqueued back to back
    # (hinv_upper_async); the last one's status is checked afterwards.
    out["inverse_factor"] = {}
    for Cf in (C, C // 4):
        Xf = torch.randn(2 * Cf, Cf, device=dev, generator=g)
        H0 = (Xf.t() @ Xf) / (2 * Cf)
        del Xf
        H = torch.empty_like(H0)
        jobs = []
        ms_copy = _ev_ms(lambda: H.copy_(H0), 3)
        ms = _ev_ms(lambda: jobs.append(kernels.hinv_upper_async(H.copy_(H0), None)), 3) - ms_copy
        _, retries, fallback = kernels.hinv_upper_finish(jobs[-1])
        fl = 2.0 * Cf ** 3 / 3
        out["inverse_factor"][f"C{Cf}"] = {
            "kernels": "k_chol_inv_node + k_sgemm/k_sgemm2 (recursive Cholesky-inverse)",
            "ms": round(ms, 3), "achieved": round(fl / ms / 1e9, 1), "peak": PEAK_F32 / 1e12,
            "unit": "TFLOP/s", "frac": round(fl / ms / 1e9 / (PEAK_F32 / 1e12), 3),
            "retries": retries, "fallback": fallback}
        del H, H0, jobs
        torch.cuda.empty_cache()
    return out


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cfg1_run(dev, method="crb"):
    """BASELINE configs[0] in full: add_batch of 16 x 512 tokens (one call per
    sequence) + fasterquant of the 768 x 768 fp32 layer, through the drop-in
    BRAGPTQ on `dev` (the crbq kernels on a GPU, or the oracle's restatement
    of the reference on the CPU).  Returns (seconds, error)."""
    W, X = synth.cfg1(0)
    if dev.type == "cpu":
        from oracle import crb_oracle as O
        t0 = time.time()
        H = torch.zeros(768, 768)
        n = 0
        for s in range(X.shape[0]):
            H, n = O.hessian_add_batch(H, n, X[s:s + 1])
        err = O.fasterquant(W, H, method=method)[2]
        return time.time() - t0, err
    import contextlib
    import io
    from crb_amd import BRAGPTQ, Binarization
    Xd = X.to(dev)
    best = None
    for _ in range(3):
        layer = torch.nn.Linear(768, 768, bias=False).to(dev)
        layer.weight.data = W.to(dev).clone()
        torch.cuda.synchronize()
        t0 = time.time()
        bq = BRAGPTQ(layer, Binarization(layer.weight, method=method, groupsize=128), "hessian")
        for s in range(Xd.shape[0]):
            bq.add_batch(Xd[s:s + 1], None)
        with contextlib.redirect_stdout(io.StringIO()):
            err = bq.fasterquant(blocksize=128, percdamp=0.01, partition=3)["error"]
        dt = time.time() - t0
        best = dt if best is None else min(best, dt)
    return best, err


def cfg2_full(dev, methods=("crb", "braq"), seed=0):
    """BASELINE configs[1] in full, on the host cores (the oracle) and on the
    GPU (the layer driver), for crb and braq: one OPT-1.3B-shaped decoder
    layer (q/k/v/out_proj 2048 x 2048, fc1 8192 x 2048, fc2 2048 x 8192,
    fp16 W ~ N(0, 0.02^2)) with 128 x 2048 fp16 tokens per distinct input
    (Student-t(4) channel scales).  The CPU side feeds one sequence per
    add_batch (run.py's hooks, bigptq.py:37-53) into one Hessian per
    distinct input, shared by the two methods as on the GPU, then runs
    fasterquant (bigptq.py:56-291) per sublayer; the GPU side runs the
    layer driver on the same tensors.  Seconds and summed errors per method
    (the two Hessians differ by summation order, so the errors agree to
    rounding unless a block's search choice sits on a near-tie)."""
    from crb_amd.driver import LayerQuantizer, Sublayer
    from oracle import crb_oracle as O
    subs = synth.opt_sublayers("opt-1.3b")
    Ws = {}
    for i, (name, r, c, grp) in enumerate(subs):
        g = torch.Generator(device=dev).manual_seed(seed * 100 + 50 + i)
        Ws[name] = (torch.randn(r, c, generator=g, device=dev) * 0.02).half()
    Cg = {grp: c for (_, _, c, grp) in subs}
    X = {}
    for j, (grp, C) in enumerate(Cg.items()):
        sc = synth.channel_scales(C, seed + 20 + j, kind="student_t4", device=dev)
        g = torch.Generator(device=dev).manual_seed(seed * 1000 + 20 + j)
        x = torch.empty(128 * 2048, C, dtype=torch.float16, device=dev)
        for t0 in range(0, x.shape[0], 8192):
            x[t0:t0 + 8192] = (torch.randn(8192, C, generator=g, device=dev) * sc).half()
        X[grp] = x
    out = {"workload": "BASELINE configs[1] in full (OPT-1.3B layer, 128x2048 fp16 tokens, "
                       "Student-t(4) channels; crb and braq, blocksize 128, hessian metric)"}
    # GPU: the layer driver, best of 2 per method
    for m in methods:
        best, errs = None, None
        for _ in range(2):
            torch.cuda.synchronize()
            t0 = time.time()
            lq = LayerQuantizer([Sublayer(n, Ws[n].clone(), gg) for (n, _, _, gg) in subs],
                                method=m)
            for grp, x in X.items():
                lq.add_batch(grp, x.view(128, 2048, -1))
            e = lq.quantize()
            torch.cuda.synchronize()
            dt = time.time() - t0
            best, errs = (dt, e) if best is None or dt < best else (best, errs)
        out[m] = {"gpu_s": round(best, 4), "gpu_error": round(sum(errs.values()), 6)}
    # CPU: the oracle
    Xc = {grp: x.cpu() for grp, x in X.items()}
    Wc = {n: w.cpu() for n, w in Ws.items()}
    del X
    torch.cuda.empty_cache()
    t0 = time.time()
    H = {}
    for grp, x in Xc.items():
        h, n = torch.zeros(Cg[grp], Cg[grp]), 0
        for s in range(128):
            h, n = O.hessian_add_batch(h, n, x[s * 2048:(s + 1) * 2048].float().unsqueeze(0))
        H[grp] = h
    t_h = time.time() - t0
    out["cpu_hessian_s"] = round(t_h, 2)
    for m in methods:
        t0 = time.time()
        err = 0.0
        for (n, _, _, grp) in subs:
            err += O.fasterquant(Wc[n], H[grp], method=m)[2]
        t_q = time.time() - t0
        out[m].update({"cpu_s": round(t_h + t_q, 2), "cpu_quantize_s": round(t_q, 2),
                       "cpu_error": round(err, 6)})
        out[m]["cpu_over_gpu"] = round(out[m]["cpu_s"] / out[m]["gpu_s"], 1)
    return out


def reference_calibration():
    """Oracle / genuine reference time ratio on configs[0], measured in the
    build container (tests/golden/time_reference.py), or None."""
    path = os.path.join(ROOT, "tests", "golden", "reference_timing.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    return {"oracle_over_reference": round(d["oracle_over_reference"], 3),
            "cpu": d["cpu"], "threads": d["threads"]}


def cpu_baseline(nseq=32, nblocks=48, cfg1_gpu=None, cfg2=None):
    """Time the test-only CPU oracle (torch-CPU restatement of the reference
    path) on a bounded sample of the workload (about 10-20 s on 16 cores)
    and extrapolate to one OPT-6.7B layer; also configs[0] in full, and
    configs[1] in full when given (cfg2_full, timed before)."""
    from oracle import crb_oracle as O
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    cfg1_cpu_s, cfg1_err = cfg1_run(torch.device("cpu"))
    C = 4096
    g = torch.Generator().manual_seed(0)
    # Hessian: nseq sequences x 2048 tokens of a 4096-channel input, fed
    # one sequence per add_batch as run.py's hooks do
    X = (torch.randn(nseq, 2048, C, generator=g) * 0.5).half()
    H = torch.zeros(C, C)
    n = 0
    t0 = time.time()
    for s in range(nseq):
        H, n = O.hessian_add_batch(H, n, X[s:s + 1].float())
    t_h = time.time() - t0
    del X
    # per layer: 128 sequences into each of the 4 distinct inputs (3 of
    # 4096 channels, 1 of 16384); the work scales with tokens * C^2
    h_layer = t_h * (128 / nseq) * (3 * 4096 ** 2 + 16384 ** 2) / 4096 ** 2
    # inverse factors: a 4096 one (x3 inputs) and an 8192 one scaled by
    # C^3 to the 16384 input
    W = torch.randn(4096, C, generator=g) * 0.02
    H += torch.eye(C) * float(H.diag().mean())
    t0 = time.time()
    O.hinv_upper(H.clone(), W.clone(), 0.01)
    t_u4 = time.time() - t0
    H8 = torch.block_diag(H, H) + 0.01 * torch.eye(2 * C)
    t0 = time.time()
    O.hinv_upper(H8, torch.zeros(1, 2 * C), 0.01)
    t_u8 = time.time() - t0
    del H8
    u_layer = 3 * t_u4 + 8 * t_u8
    # block loop: the first nblocks CRB blocks of a 4096 x 4096 sublayer;
    # a layer has sum(R*C)/128 = 1.57M row-blocks, the sample nblocks*4096
    t0 = time.time()
    O.fasterquant(W, H, method="crb", max_blocks=nblocks)
    t_b = time.time() - t0 - t_u4   # fasterquant recomputes the factor
    rowblocks = (4 * 4096 * 4096 + 2 * 4096 * 16384) / 128
    b_layer = max(t_b, 0.0) / (nblocks * 4096) * rowblocks
    total = h_layer + u_layer + b_layer
    return {
        "value": total, "unit": "s/layer", "cores": ncores, "kind": "port",
        "sample": (f"oracle (torch-CPU restatement of bigptq/binary/utils) on this host, "
                   f"{t_h + t_u4 + t_u8 + t_b + t_u4:.1f}s of CPU work: Hessian of {nseq}x2048 "
                   f"tokens x 4096 ch ({t_h:.2f}s), inverse factors of a 4096 and an 8192 "
                   f"Hessian ({t_u4:.2f}s, {t_u8:.2f}s), first {nblocks} CRB blocks of a "
                   f"4096x4096 sublayer ({t_b:.2f}s); extrapolated to one OPT-6.7B layer by "
                   f"token count, C^3 and row-blocks"),
        "split_s": {"hessian": h_layer, "hinv": u_layer, "blocks": b_layer},
        "cfg1_full": {"workload": "BASELINE configs[0] in full (768x768 fp32, 16x512 tokens, "
                                  "crb)", "cpu_s": round(cfg1_cpu_s, 3),
                      "cpu_error": cfg1_err,
                      "gpu_s": None if cfg1_gpu is None else round(cfg1_gpu[0], 4),
                      "gpu_error": None if cfg1_gpu is None else cfg1_gpu[1]},
        "cfg2_full": cfg2,
        "calibration": reference_calibration(),
        "cpu": cpu_model(),
        "blas": torch.__config__.show().split("BLAS_INFO=")[-1].split(",")[0]
        if "BLAS_INFO=" in torch.__config__.show() else "unknown",
    }


def syrk_compare(dev, ntok, reps=2):
    """The fc2 input's Hessian product two ways on the same data, for counter
    runs that compare them kernel by kernel: crbq_hessian_accum (transpose
    into the channel-major copy + k_syrk16k_pers over the upper triangle) and
    hipBLASLt (torch.mm, fp16 in / fp32 accumulate / fp16 out) on the same
    channel-major operand, the full C x C product.  Each timed with events
    on the current stream; prints TFLOP/s of the symmetric half T C (C + 1)
    for ours and of the full 2 T C^2 for the library."""
    from crb_amd import kernels
    C = 16384
    X = make_inputs(dev, ntok)["fc2"]
    S = torch.zeros(C, C, device=dev)
    res = {}
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    for r in range(reps):
        S.zero_()
        ev[0].record()
        kernels.hessian_accum(X, S)
        ev[1].record()
        torch.cuda.synchronize()
        res.setdefault("crbq_hessian_accum_ms", []).append(round(ev[0].elapsed_time(ev[1]), 3))
    del S
    Xt = X.t().contiguous()
    del X
    torch.cuda.empty_cache()
    for r in range(reps):
        ev[0].record()
        P = torch.mm(Xt, Xt.t())
        ev[1].record()
        torch.cuda.synchronize()
        res.setdefault("torch_mm_channel_major_ms", []).append(round(ev[0].elapsed_time(ev[1]),
                                                                     3))
        del P
    t_ours = min(res["crbq_hessian_accum_ms"]) / 1e3
    t_lib = min(res["torch_mm_channel_major_ms"]) / 1e3
    res["crbq_TFLOP_s_symmetric"] = round(ntok * C * (C + 1) / t_ours / 1e12, 1)
    res["torch_mm_TFLOP_s_full"] = round(2 * ntok * C * C / t_lib / 1e12, 1)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--method", default="crb")
    ap.add_argument("--tokens", type=int, default=128 * 2048)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-packed", action="store_true", help="skip the packed GEMV timing")
    ap.add_argument("--stack-layers", type=int, default=32,
                    help="layers of the OPT-6.7B-shaped stack run (0: skip); the default "
                         "is the whole 32-layer stack of BASELINE configs[2]")
    ap.add_argument("--fc2-last", action="store_true",
                    help="accumulate the fc2 input's Hessian last (forward order)")
    ap.add_argument("--no-kernels", action="store_true",
                    help="skip the block loop's isolated kernel measurements")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the block loop's kernels against their rooflines (the "
                         "'kernels' object), for counter runs of those kernels")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only copy a 1 GiB buffer 3 times: the known-size copy kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE for the traffic figure")
    ap.add_argument("--no-cfg2-full", action="store_true",
                    help="skip configs[1] in full (OPT-1.3B layer, crb and braq, oracle on "
                         "the host cores and the GPU) in the CPU baseline")
    ap.add_argument("--syrk-compare", action="store_true",
                    help="only the fc2 input's Hessian product through the library and "
                         "through hipBLASLt (torch.mm) on the same channel-major data, for "
                         "counter runs comparing the two kernels")
    ap.add_argument("--packed-only", action="store_true",
                    help="only the packed GEMV / GEMM timing (the 'packed_gemv' object), for "
                         "counter runs of those kernels")
    args = ap.parse_args()
    if args.packed_only:
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        print(json.dumps({"packed_gemv": packed_gemv(dev)}))
        return
    if args.syrk_compare:
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        print(json.dumps({"syrk_compare": syrk_compare(dev, args.tokens)}))
        return
    if args.calibrate_copy:
        x = torch.ones(256 * 1024 * 1024, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": x.numel() * 4, "copies": 3}))
        return
    if args.kernels_only:
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        print(json.dumps({"kernels": kernel_rooflines(dev)}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the path would shard "
                                   "by sublayer and by calibration tokens, but no "
                                   "multi-GPU figure is produced"}))
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from crb_amd import _lib
    _lib.ready(dev)
    bin_rates = None
    if not args.no_kernels:
        # the standalone binarizer first, on a chip that has not yet run the
        # layer at its power limit (kernel_rooflines measures it again after)
        bin_rates = binarize_rates(dev)
        print(f"[bench] binarizer: {bin_rates}", file=sys.stderr, flush=True)
    print(f"[bench] building OPT-6.7B layer inputs ({args.tokens} tokens)", file=sys.stderr,
          flush=True)
    subs, W0 = make_layer(dev)
    X = make_inputs(dev, args.tokens, fc2_first=not args.fc2_last)
    torch.cuda.synchronize()
    for w in range(args.warmup):
        one_layer(subs, W0, X, args.method, timing=False)
        torch.cuda.synchronize()
        print(f"[bench] warmup {w} done", file=sys.stderr, flush=True)
    from crb_amd import kernels
    torch.cuda.synchronize()
    kernels.syrk_timing_collect()
    # the library brackets every SYRK kernel launch with HIP events on the
    # stream it is launched on
    kernels.syrk_timing(True)
    t0 = time.time()
    for k in range(args.steps):
        one_layer(subs, W0, X, args.method, timing=False)
    torch.cuda.synchronize()
    dt = (time.time() - t0) / args.steps
    kernels.syrk_timing(False)
    print(f"[bench] timed {args.steps} steps: {dt:.4f} s/layer", file=sys.stderr, flush=True)
    # dominant kernel: the Hessian SYRK of the fc2 input (C = 16384), one
    # launch per step; its duration is averaged over the timed steps
    T = args.tokens
    Cfc2 = 16384
    fc2_ms = [ms for (c, ms) in kernels.syrk_timing_collect() if c == Cfc2]
    assert len(fc2_ms) == args.steps, fc2_ms
    flops = T * Cfc2 * (Cfc2 + 1)
    t_launch = sum(fc2_ms) / len(fc2_ms) / 1e3
    achieved = flops / t_launch
    # phase split (separate, instrumented step)
    lq, pt = one_layer(subs, W0, X, args.method, timing=True)
    torch.cuda.synchronize()
    h_ms = {g: lq.syrk_ms(g) for g in X}
    hess_ms = sum(h_ms.values())
    cols = sum(c for (_, r, c, _) in subs)
    out = {
        "metric": METRIC, "value": round(dt, 5), "unit": "s/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 in / fp32 accumulate+quantize", "data": "synthetic",
        "config": {"workload": "OPT-6.7B decoder layer (BASELINE configs[2], per layer)",
                   "method": args.method, "blocksize": 128, "salient_metric": "hessian",
                   "tokens": T, "sublayers": [n for (n, _, _, _) in subs]},
        "cols_per_s": round(cols / dt, 1),
        "phase_ms": {"hessian": round(hess_ms, 3),
                     "quantize_overlapped": round(pt.quantize_ms, 3),
                     "hinv": {g: round(v, 3) for g, v in pt.hinv_ms.items()},
                     "factor_plus_blocks": {g: round(v, 3) for g, v in pt.chain_ms.items()}},
        "roofline": {"bound": "mfma",
                     "kernel": "k_syrk16k_pers<TM> (Hessian SYRK, token-major stages, "
                               "fc2 input C=16384)",
                     "achieved": round(achieved / 1e12, 2), "peak": PEAK_F16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_F16, 4),
                     "launch_ms": round(t_launch * 1e3, 3),
                     "algorithmic_flop": flops,
                     "traffic": load_traffic("syrk_fc2_opt67b_traffic.md")},
    }
    pv = load_profile_values("mfma_busy_layer.md") or {}
    if "syrk_fc2_mfma_busy_per_simd" in pv:
        # rocprofv3 counters of the same kernel: matrix-unit busy fraction
        # and the engine clock it ran at (quoted peaks assume 2.4 GHz)
        out["roofline"]["mfma_busy_per_simd"] = pv["syrk_fc2_mfma_busy_per_simd"]
        out["roofline"]["clock_ghz_under_load"] = pv.get("syrk_fc2_clock_ghz")
    # The operand stream from L2 into LDS: every upper 256 x 256 tile loads
    # both 256-channel panels (2 x 256 x 2 bytes per token), 1/64 byte per
    # multiply-add; at full MFMA rate a CU would need 32 bytes per clock.
    # The chip holds 1.6-1.75 GHz under this stream (the kernel without its
    # loads runs at 2.0 GHz); hipBLASLt's 256 x 256 kernel on the same
    # operand streams 28.8 B/clk/CU at 90 % MFMA busy and 1.46 GHz.
    nt = (Cfc2 + 255) // 256
    sbytes = nt * (nt + 1) // 2 * 2 * 256 * 2 * T
    stream = {"bytes": sbytes, "achieved_TB_s": round(sbytes / t_launch / 1e12, 2)}
    clk = out["roofline"].get("clock_ghz_under_load")
    if clk:
        stream["bytes_per_clk_per_cu"] = round(sbytes / t_launch / 256 / (clk * 1e9), 1)
    out["roofline"]["operand_stream_l2_to_lds"] = stream
    if not args.no_kernels:
        out["kernels"] = kernel_rooflines(dev, binarize=bin_rates)
        print(f"[bench] kernels: {out['kernels']}", file=sys.stderr, flush=True)
    if args.stack_layers > 0:
        del X
        torch.cuda.empty_cache()
        print(f"[bench] stack run, {args.stack_layers} layers", file=sys.stderr, flush=True)
        out["with_capture"] = stack_run(dev, args.stack_layers, args.tokens)
        print(f"[bench] stack: {out['with_capture']}", file=sys.stderr, flush=True)
    if not args.no_packed:
        out["packed_gemv"] = packed_gemv(dev)
        print(f"[bench] packed gemv: {out['packed_gemv']}", file=sys.stderr, flush=True)
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        cfg2 = None
        if not args.no_cfg2_full:
            cfg2 = cfg2_full(dev)
            print(f"[bench] configs[1] in full: {cfg2}", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(cfg1_gpu=cfg1_run(dev), cfg2=cfg2)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
