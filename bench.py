"""Benchmark of the int8 GEMM hot path on one MI355X.

Workload (the shape the metric's 60 %-of-peak target names): cuPOW
NoisyGEMM mining at m = n = k = 4096, rank r = 64 with the reference's noise rules, one step =
one nonce = the full useful mined forward of MinedWeight (commit A, noise, projections, hashed
noisy GEMM with every 8 x 16 tile digested, exact denoise, int32 output). B and its block-side
noise are prepared once (setup_block); the per-nonce A_i are seeded, distinct and resident in
HBM before the timed region.

value = whole-job int8 TOPS = 2 m n k * steps / time (the reference's convention,
miner/ampere/bench/bench_gemm.py:37-56). The line also carries:
  roofline      the noisy GEMM kernel alone, timed with HIP events on its launch stream inside
                the timed loop: algorithmic ops = 2 m n k + 2 m n (2 r) L (main + denoise MFMA
                work) per launch / its average duration, against 5.0 POP/s dense int8;
  detrt_layer   BASELINE configs[1]: the four linears of a Qwen3-1.7B layer at M = 2048
                (quant_act -> exact GEMM -> fused dequant), TOPS of the GEMMs;
  detrt_skinny  BASELINE configs[0] (64 x 2048 -> 6144) and configs[3]'s decode shapes (Llama-3.1-8B
                linears at M = 1, 8, 32): device time from graph replays over > 1.2 GB of rotated
                weights, algorithmic bytes / time against 8 TB/s HBM;
  llama_prefill configs[3]'s prefill shapes (M = 8192), TOPS of the four GEMMs;
  qwen3_e2e     configs[4]: the 28-layer Qwen3-1.7B-shaped integer forward over 8192 tokens (all
                decoder-layer ops, per-layer stage-output roots and the lm_head logits on the GPU),
                with a T = 64 parity check against the CPU oracle and a CPU baseline;
  cpu_baseline  the CPU oracle (this repo's C restatement, OpenMP) on a bounded sample of the
                same workload: full mined forwards of whole nonces at the same shape;
  parity        the sampled nonce's GPU output, every tile digest and the winner set compared
                with the CPU oracle, bit for bit.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "useful-work-coin_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "int8 TOPS & % of MI355X int8 MFMA peak (NoisyGEMM, detrt linear), bit-exact"
PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """The host the CPU baselines ran on: the CPU model (lscpu, else /proc/cpuinfo), os.cpu_count()
    and the cores this process may run on."""
    model = None
    try:
        import subprocess
        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except Exception:
        model = None
    if model is None:
        try:
            with open("/proc/cpuinfo") as f:
                model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), None)
        except OSError:
            model = None
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = None
    return dict(cpu_model=model, cpu_count=os.cpu_count(), cpus_available=avail)


def mfma_ceiling(torch):
    """Sustained int8 MFMA rate of the part (uwc_mfma_rate_probe: a register-only MFMA loop on every
    SIMD), with constant and with random operands, in TOP/s. The random-operand rate is the
    power-limited ceiling for a GEMM on real data."""
    from uwc_amd import _lib
    L = _lib.lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(cus * 512, dtype=torch.int32, device="cuda")
    iters = 20000
    ops_per_launch = cus * 8.0 * iters * 8 * 65536
    out = {}
    for name, rnd in (("constant_operands", 0), ("random_operands", 1)):
        f = lambda: L.uwc_mfma_rate_probe(iters, rnd, sink.data_ptr(), sink.numel(),  # noqa: E731
                                          torch.cuda.current_stream().cuda_stream)
        assert f() == 0
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            f()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(ops_per_launch * 3 / (e0.elapsed_time(e1) * 1e-3) / 1e12, 1)
    log(f"mfma ceiling: {out}")
    return out


def mining(args, torch, np, ops):
    dev = "cuda"
    m = n = k = args.size
    r = args.rank
    rng = np.random.default_rng(2026)
    Bt = torch.from_numpy(rng.integers(-64, 64, size=(n, k), dtype=np.int8)).to(dev)
    job_key = rng.bytes(32)
    target = ops.bound_words(((1 << 256) - 1) * 12 // ((m // 8) * (n // 16)))  # about 12 winning 8 x 16 tiles
    # win records: about 12 winners per nonce are expected; 256 record slots per nonce (the count
    # itself is exact beyond the cap, as in the reference's buffers)
    w = ops.MinedWeight(Bt=Bt, b_scale=torch.ones(n, device=dev), r=r, max_wins=256)
    w.setup_block(job_key, target)
    nA = args.steps + args.warmup
    nbuf = min(nA, args.distinct)
    gen = torch.Generator(device=dev)
    As = []
    for i in range(nbuf):
        gen.manual_seed(1000 + i)
        As.append(torch.randint(-64, 64, (m, k), dtype=torch.int8, device=dev, generator=gen))
    ones = torch.ones(m, device=dev)
    # distinct int32 outputs rotated through the sweep (64 MiB each at 4096^2): together larger than
    # the 256 MB Infinity Cache, so the outputs' write-back is paid as in a real sweep
    outbufs = [torch.empty((m, n), dtype=torch.int32, device=dev) for _ in range(args.out_buffers)]
    rot = lambda count, first=0: [outbufs[(first + i) % len(outbufs)] for i in range(count)]  # noqa: E731
    torch.cuda.synchronize()
    log(f"mining: {m}x{n}x{k} r={r}, {nbuf} distinct A resident, {len(outbufs)} output buffers, warmup "
        f"{args.warmup}, steps {args.steps}")

    # the sweep runs through MinedWeight.forward_many: one batched commitment and one noise launch
    # per group of nonces, then each nonce's projections and hashed GEMM
    # the warm-up covers at least two groups: forward_many alternates two sets of workspace slots,
    # which it allocates on first use
    # On a box whose GPU and host cores have been idle, the first sweeps ran up to 1.7x slower (the
    # GEMM alone 6%): warm-up sweeps repeat until both the nonce count and the time are reached,
    # and the JSON line reports the nonces actually run.
    nwarm = max(args.warmup, 2 * args.group)
    warm_list = [As[i % nbuf] for i in range(nwarm)]
    w.reserve_sweep(m, max(nwarm, args.steps))  # the sweep's win rows (device + pinned host), allocated before timing
    done, tw = 0, time.perf_counter()
    while done < args.warmup or done < 2 * args.group or time.perf_counter() - tw < args.warmup_seconds:
        w.forward_many(warm_list, ones, outs=rot(nwarm, done), out_mode=ops.OUT_I32, group=args.group,
                       gemm_group=args.gemm_group)
        torch.cuda.synchronize()
        done += nwarm
    args.warmup_nonces_run = done
    log(f"mining: warm-up {done} nonces in {time.perf_counter() - tw:.2f} s")
    sweep = [As[(done + i) % nbuf] for i in range(args.steps)]
    t0 = time.perf_counter()
    w.forward_many(sweep, ones, outs=rot(args.steps), out_mode=ops.OUT_I32, group=args.group,
                   gemm_group=args.gemm_group)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sweep_wins = w.sweep_winners()  # every nonce's winners, read back group by group during the sweep

    # the noisy GEMM alone: HIP events on its stream around back-to-back launches of the sweep's
    # last batched GEMM call (one launch = one group of nonces: same operands, corrections, seeds
    # and target). No events sit inside the sweep: recording one costs the host ~0.2 ms, more than
    # a nonce's GPU time.
    w.forward_many(sweep[-args.group:], ones, outs=rot(args.group), out_mode=ops.OUT_I32, group=args.group,
                   gemm_group=args.gemm_group)
    per_launch, relaunch = w.last_gemm_launch()
    reps = gemm_reps(args.steps)
    for _ in range(2):
        relaunch()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gc.disable()  # as forward_many does: no collection pause may starve the GPU between launches
    try:
        e0.record()
        for _ in range(reps):
            relaunch()
        e1.record()
        torch.cuda.synchronize()
    finally:
        gc.enable()
    dt = t1 - t0
    launch_ms = e0.elapsed_time(e1) / reps
    kern_ms = launch_ms / per_launch  # per nonce
    b = w._buf(m, slot=1)  # forward_many's first slot: an item of the last group
    mx = int(b["maxabs"].max().item())
    L = ops.limbs_for_max(mx)
    ops_main = 2.0 * m * n * k
    ops_kernel = ops_main + 2.0 * m * n * 2 * r * L
    tops = ops_main * args.steps / dt / 1e12
    kern_tops = ops_kernel / (kern_ms * 1e-3) / 1e12
    log(f"mining: {dt * 1e3 / args.steps:.3f} ms/nonce, {tops:.1f} TOPS whole path; noisy_gemm {launch_ms * 1e3:.1f} us "
        f"per launch of {per_launch} nonces = {kern_ms * 1e3:.1f} us per nonce = {kern_tops:.1f} TOP/s (L={L})")
    res = dict(m=m, n=n, k=k, r=r, dt=dt, tops=tops, kern_ms=kern_ms, kern_tops=kern_tops, L=L, w=w, As=As,
               launch_ms=launch_ms, per_launch=per_launch, sweep_winners=sum(len(x) for x in sweep_wins),
               job_key=job_key, target=target, Bt=Bt, ones=ones)
    return res


def noise_mining(args, torch, np, ops):
    """Pure noise mining at the reference miner's shape (miner_loop.py:35-38): m = 8192, n = 16384,
    k = 4096, r = 128; per attempt MinedWeight.noise_mine (commit A, noise, noised A, hashed GEMM
    with every tile digested, no output), over resident random A rotated through 4 buffers. The
    reference's sustained figures for this loop are 70-73 hashed TMAC/s on an RTX 3080 and 320-330
    on an RTX 5090 (spec/step1-results.md:39-40, 141; results/matrix_q4.txt:5,10)."""
    dev = "cuda"
    m, n, k, r = 8192, 16384, 4096, 128
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    Bt = torch.randint(-64, 65, (n, k), dtype=torch.int8, device=dev, generator=gen)
    w = ops.MinedWeight(Bt=Bt, b_scale=torch.ones(n, device=dev), r=r, max_wins=64)
    w.setup_block(bytes(range(32)), ops.bound_words(((1 << 256) - 1) * 4 // ((m // 8) * (n // 16))))
    As = [torch.randint(-64, 65, (m, k), dtype=torch.int8, device=dev, generator=gen) for _ in range(4)]
    for i in range(4):
        w.noise_mine(As[i % 4])
    torch.cuda.synchronize()
    attempts, t0 = 0, time.perf_counter()
    while attempts < args.mine_attempts or time.perf_counter() - t0 < 1.0:
        for i in range(8):
            w.noise_mine(As[(attempts + i) % 4])
        attempts += 8
        torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    wins = len(w.winners(m))
    tmacs = m * n * k * attempts / dt / 1e12
    out = dict(workload=f"noise_mine {m}x{n}x{k} r={r}: commitment + noise + noised A + hashed GEMM per attempt",
               attempts=attempts, ms_per_attempt=round(dt * 1e3 / attempts, 4), hashed_tmacs=round(tmacs, 1),
               int8_tops=round(2 * tmacs, 1), last_attempt_winners=wins,
               reference_tmacs={"rtx3080": [70, 73], "rtx5090": [320, 330]})
    log(f"noise mining: {out}")
    return out


def parity_and_cpu(args, res, torch, np, ops, O):
    """Re-run one group of the sweep on the GPU, through the same batched split-role GEMM launch the
    sweep and the roofline time, with a tile dump per nonce, and compare its first nonce with the
    oracle (output, every tile message and digest, winners), timing the oracle's full mined
    forward of that nonce on the host."""
    m, n, k, r = res["m"], res["n"], res["k"], res["r"]
    w = res["w"]
    group = [res["As"][i % len(res["As"])] for i in range(args.gemm_group)]
    dumps = [torch.zeros((m // 64) * 8 * (n // 64) * 4 * ops.DUMP_WORDS, dtype=torch.int32, device="cuda")
             for _ in group]
    outs = w.forward_many(group, res["ones"], out_mode=ops.OUT_I32, group=args.group, gemm_group=args.gemm_group,
                          dumps=dumps)
    torch.cuda.synchronize()
    wins = set(w.sweep_winners()[0])
    out, dump, A = outs[0], dumps[0], group[0]
    A_np = A.cpu().numpy()
    Bt_np = res["Bt"].cpu().numpy()
    blk = O.block_side(res["job_key"], Bt_np, r)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    t0 = time.perf_counter()
    nonces = 0
    ref = None
    while True:
        ref_i = O.mined_forward(A_np, Bt_np, res["job_key"], res["target"], r, blk=blk)
        ref = ref if ref is not None else ref_i
        nonces += 1
        if time.perf_counter() - t0 >= args.cpu_seconds or nonces >= args.cpu_max_nonces:
            break
    t_cpu = time.perf_counter() - t0
    d = dump.cpu().numpy().view(np.uint32).reshape(m // 64, 8, n // 64, 4, ops.DUMP_WORDS)
    parity = dict(kernel="noisy_gemm256_kernel<true, true, 1, true> (the timed split launch)",
                  nonces_in_launch=len(group), nonces_checked=1,
                  output_exact=bool(np.array_equal(out.cpu().numpy(), ref["out"])),
                  tile_digests_equal=bool(np.array_equal(d[..., 16:], ref["digests"])),
                  tile_messages_equal=bool(np.array_equal(d[..., :16], ref["msgs"])),
                  winners_equal=bool(wins == ref["winners"]), winners=len(wins),
                  tiles=int(d.shape[0] * 8 * d.shape[2] * 4))
    cpu = dict(value=round(2.0 * m * n * k * nonces / t_cpu / 1e12, 4), unit="TOPS", cores=threads, kind="port", **host_cpu(),
               sample=f"{nonces} full mined forward(s) (commit, noise, projections, transcript of every tile, "
                      f"digests, denoise) at {m}x{n}x{k} r={r}, {t_cpu:.1f} s, oracle/uwc_oracle.c with {threads} "
                      f"OpenMP threads")
    log(f"cpu oracle: {nonces} nonce(s) in {t_cpu:.1f} s; parity {parity}")
    return parity, cpu


def detrt_layer(args, torch, np):
    """qkv, o, gu, down of a Qwen3-1.7B layer at M = 2048 through DetLinear.
    Device time: the four calls (quant_act + exact GEMM with fused dequant each) captured in a HIP
    graph and replayed; beside it the GEMM-only time (the four uwc_igemm_dequant_f32 launches on
    pre-quantized activations, graph-replayed) and the host-timed eager figure."""
    from uwc_amd import _lib, detrt
    dev = "cuda"
    L = _lib.lib()
    M, D, I, H, Hkv, hd = 2048, 2048, 6144, 16, 8, 128
    shapes = {"qkv": ((H + 2 * Hkv) * hd, D), "o": (D, H * hd), "gu": (2 * I, D), "down": (D, I)}
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    lays, xs = {}, {}
    for name, (nn, kk) in shapes.items():
        W = torch.randn((nn, kk), device=dev, generator=g) * 0.02
        lays[name] = detrt.DetLinear(W, dev, 512)
        xs[name] = torch.randn((M, kk), device=dev, generator=g)
    for name in shapes:
        lays[name](xs[name])
    torch.cuda.synchronize()
    macs = sum(M * nn * kk for nn, kk in shapes.values())
    # host-timed eager calls (launch overhead included)
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        for name in shapes:
            lays[name](xs[name])
    torch.cuda.synchronize()
    host_dt = (time.perf_counter() - t0) / reps
    # device time of the whole linears: one graph of the four DetLinear calls
    keep = []

    def call(name):
        keep.append(lays[name](xs[name]))
        return 0
    layer_us = _graph_time_us(torch, [lambda nm=nm: call(nm) for nm in shapes]) * len(shapes)
    keep.clear()
    # GEMM-only device time per linear
    stream_of = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    gemm_us, per = 0.0, {}
    vend = dict(ours=0.0, blas=0.0, equal=True)
    for name, (nn, kk) in shapes.items():
        q, sx = detrt.quant_act(xs[name], lays[name].bs)
        y = torch.empty((M, nn), dtype=torch.float32, device=dev)
        lay = lays[name]
        f = lambda q=q, sx=sx, y=y, lay=lay, nn=nn, kk=kk: L.uwc_igemm_dequant_f32(  # noqa: E731
            q.data_ptr(), lay.Wq.data_ptr(), M, nn, kk, sx.data_ptr(), lay.sw.data_ptr(), y.data_ptr(), stream_of())
        us = _graph_time_us(torch, [f] * 8)
        o_us, b_us, same = vendor_i32(torch, L, q, lay.Wq)
        per[name] = dict(us=round(us, 2), tops=round(2.0 * M * nn * kk / us / 1e6, 1), i32_us=round(o_us, 2),
                         hipblaslt_i32_us=round(b_us, 2), hipblaslt_equal=same)
        gemm_us += us
        vend["ours"] += o_us
        vend["blas"] += b_us
        vend["equal"] &= same
    import oracle as O
    ctops, ct, ran, cores = cpu_linears(torch, np, O, M, shapes, budget_s=3.0)
    out = dict(workload="Qwen3-1.7B layer linears (qkv, o, gu, down) at M=2048, quant_act + exact GEMM + dequant",
               ms_per_layer=round(layer_us / 1e3, 4), tops=round(2.0 * macs / layer_us / 1e6, 2),
               frac_of_peak=round(2.0 * macs / layer_us / 1e6 / PEAK_INT8_TOPS, 4),
               timing="device (HIP graph of the four DetLinear calls, replayed)",
               gemm_only=dict(us_per_layer=round(gemm_us, 2), tops=round(2.0 * macs / gemm_us / 1e6, 1),
                              frac_of_peak=round(2.0 * macs / gemm_us / 1e6 / PEAK_INT8_TOPS, 4), per_linear=per,
                              kernel="uwc_igemm_dequant_f32 (exact int8 GEMM, fused fp32 dequant), graph-replayed"),
               vs_hipblaslt=dict(ours_i32_us_per_layer=round(vend["ours"], 2),
                                 hipblaslt_i32_us_per_layer=round(vend["blas"], 2), outputs_equal=vend["equal"],
                                 note="the four GEMMs on the same int8 operands, int32 out: uwc_igemm_i32 against "
                                      "torch._int_mm (hipBLASLt), graph-replayed on this box"),
               host_ms_per_layer=round(host_dt * 1e3, 4),
               cpu_baseline=dict(value=round(ctops, 4), unit="TOPS", cores=cores, kind="port", **host_cpu(),
                                 sample=f"quant_act + fp64 matmul + dequant, {ran}, {ct:.2f} s"))
    log(f"detrt layer: {out}")
    return out


def _graph_time_us(torch, launches, reps=3):
    """Average device time per launch of a list of zero-argument launch closures, captured once
    into a HIP graph and replayed (so host launch overhead is not measured), HIP events on the
    capturing stream."""
    for f in launches:  # eager warm-up: one-time attribute setup happens outside the capture
        assert f() == 0, "launch failed"
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for f in launches:
                assert f() == 0, "launch failed during capture"
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(launches))


def vendor_i32(torch, L, A, W):
    """The same int8 GEMM on the same operands, int32 out, two ways, graph-replayed: this library's
    uwc_igemm_i32 and the vendor's (torch._int_mm, hipBLASLt on ROCm). Returns (ours_us, blas_us,
    outputs_equal)."""
    m, k = A.shape
    n = W.shape[0]
    C = torch.empty((m, n), dtype=torch.int32, device=A.device)
    Wt = W.t()  # k x n, column-major: the layout _int_mm takes for A W^T
    ours = lambda: L.uwc_igemm_i32(A.data_ptr(), W.data_ptr(), m, n, k, C.data_ptr(),  # noqa: E731
                                   torch.cuda.current_stream().cuda_stream)
    ours_us = _graph_time_us(torch, [ours] * 4)
    blas_us = _graph_time_us(torch, [lambda: (torch._int_mm(A, Wt), 0)[1]] * 4)
    torch.cuda.synchronize()
    same = bool(torch.equal(torch._int_mm(A, Wt), C))
    del C
    return ours_us, blas_us, same


def cpu_linears(torch, np, O, m, shapes, budget_s=3.0):
    """The reference's CPU path for detrt linears, restated: quant_act (oracle) -> the fp64 matmul
    q.double() @ Wq.double().T (runtime/detrt/qwen3.py:109-110) -> dequant (oracle), with torch using
    every host core as runtime/bench/xdevice.py:28 does. Runs the listed linears once each
    (after a small warm-up) unless that exceeds budget_s, then extrapolates from the linears run.
    Returns (TOPS of the GEMMs, seconds, what was run)."""
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    rng = np.random.default_rng(11)
    xw = torch.from_numpy(rng.integers(-64, 65, size=(8, 64)).astype(np.float64))
    xw @ xw.T
    ops_done, t_done, ran, ops_all = 0.0, 0.0, [], 0.0
    for name, (n, k) in shapes.items():
        ops_all += 2.0 * m * n * k
        if t_done > budget_s:
            continue
        x = rng.standard_normal((m, k)).astype(np.float32)
        Wq = torch.from_numpy(rng.integers(-64, 65, size=(n, k), dtype=np.int8))
        sw = rng.random(n, dtype=np.float32)
        t0 = time.perf_counter()
        q, sx = O.quant_act(x, 512 if k % 512 == 0 else 0)
        acc = (torch.from_numpy(q).double() @ Wq.double().T).numpy().astype(np.int32)
        O.dequant(acc, sx, sw)
        t_done += time.perf_counter() - t0
        ops_done += 2.0 * m * n * k
        ran.append(name)
    tops = ops_done / t_done / 1e12
    return tops, t_done, ran, threads


def _weight_copies(wb):
    """Distinct weight buffers a skinny shape rotates over: > 1.2 GB in all, at least 2."""
    return max(2, -(-(1200 << 20) // wb))


def _skinny_launches(wb, reps_cap=48):
    """Launches in a skinny shape's timing graph."""
    return min(max(2 * _weight_copies(wb), 16), reps_cap)


LLAMA_LINEARS = {"qkv": (6144, 4096), "o": (4096, 4096), "gu": (28672, 4096), "down": (4096, 14336)}


def skinny_linears(args, torch, np):
    """BASELINE configs[0] (detrt MLP-up, 64 x 2048 -> 6144) and the decode half of configs[3]
    (Llama-3.1-8B layer linears at M = 1, 8, 32): exact GEMM + fused fp32 dequant through
    uwc_igemm_dequant_f32, weights rotated over > 1.2 GB of distinct buffers so the 256 MB
    Infinity Cache cannot serve them. Algorithmic bytes = W + X + fp32 out + scales; roofline =
    those bytes / device time vs 8 TB/s."""
    from uwc_amd import _lib
    dev = "cuda"
    L = _lib.lib()
    stream_of = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def run(m, shapes, reps_cap=48):
        """time per layer (sum over shapes) for token count m."""
        total_us, total_bytes, per = 0.0, 0, {}
        for name, (n, k) in shapes.items():
            wb = n * k
            nw = _weight_copies(wb)
            Ws = [torch.randint(-64, 65, (n, k), dtype=torch.int8, device=dev) for _ in range(nw)]
            X = torch.randint(-64, 65, (m, k), dtype=torch.int8, device=dev)
            sx, sw = torch.rand(m, device=dev) + 0.5, torch.rand(n, device=dev) * 1e-3
            Y = torch.empty((m, n), dtype=torch.float32, device=dev)

            def mk(W):
                return lambda: L.uwc_igemm_dequant_f32(X.data_ptr(), W.data_ptr(), m, n, k, sx.data_ptr(),
                                                       sw.data_ptr(), Y.data_ptr(), stream_of())
            launches = [mk(Ws[i % nw]) for i in range(_skinny_launches(wb, reps_cap))]
            us = _graph_time_us(torch, launches)
            byt = wb + m * k + 4 * m * n + 4 * (m + n)
            per[name] = dict(us=round(us, 2), gbs=round(byt / us / 1e3, 1))
            total_us += us
            total_bytes += byt
            del Ws
            torch.cuda.empty_cache()
        return total_us, total_bytes, per

    import oracle as O
    out = {}
    us, byt, per = run(64, {"mlp_up": (6144, 2048)})
    ctops, ct, ran, cores = cpu_linears(torch, np, O, 64, {"mlp_up": (6144, 2048)})
    out["config1_mlp_up_64x2048x6144"] = dict(
        us=round(us, 2), bytes=byt, gbs=round(byt / us / 1e3, 1), hbm_frac=round(byt / us / 1e3 / PEAK_HBM_GBS, 4),
        tops=round(2.0 * 64 * 6144 * 2048 / us / 1e6, 2),
        cpu_baseline=dict(value=round(ctops, 4), unit="TOPS", cores=cores, kind="port", **host_cpu(),
                          sample=f"quant_act + fp64 matmul + dequant, {ran}, {ct:.2f} s"))
    llama = LLAMA_LINEARS
    dec = {}
    for m in (1, 8, 32):
        us, byt, per = run(m, llama)
        ctops, ct, ran, cores = cpu_linears(torch, np, O, m, llama, budget_s=2.0)
        dec[f"M{m}"] = dict(us_per_layer=round(us, 2), bytes_per_layer=byt, gbs=round(byt / us / 1e3, 1),
                            hbm_frac=round(byt / us / 1e3 / PEAK_HBM_GBS, 4), per_linear=per,
                            cpu_baseline=dict(value=round(ctops, 5), unit="TOPS", cores=cores, kind="port", **host_cpu(),
                                              sample=f"quant_act + fp64 matmul + dequant, {ran}, {ct:.2f} s"))
    out["config4_llama8b_decode"] = dec
    log(f"skinny linears: {json.dumps(out)}")
    return out


def llama_prefill(args, torch, np):
    """The prefill half of BASELINE configs[3]: Llama-3.1-8B layer linears at M = 8192, exact
    GEMM + fused fp32 dequant (uwc_igemm_dequant_f32), TOPS of the four GEMMs."""
    from uwc_amd import _lib
    dev = "cuda"
    L = _lib.lib()
    M = 8192
    shapes = {"qkv": (6144, 4096), "o": (4096, 4096), "gu": (28672, 4096), "down": (4096, 14336)}
    per, total_us, ops = {}, 0.0, 0.0
    vend = dict(ours=0.0, blas=0.0, equal=True)
    for name, (n, k) in shapes.items():
        X = torch.randint(-64, 65, (M, k), dtype=torch.int8, device=dev)
        W = torch.randint(-64, 65, (n, k), dtype=torch.int8, device=dev)
        sx, sw = torch.rand(M, device=dev), torch.rand(n, device=dev)
        Y = torch.empty((M, n), dtype=torch.float32, device=dev)
        f = lambda: L.uwc_igemm_dequant_f32(X.data_ptr(), W.data_ptr(), M, n, k, sx.data_ptr(), sw.data_ptr(),  # noqa: E731
                                            Y.data_ptr(), torch.cuda.current_stream().cuda_stream)
        us = _graph_time_us(torch, [f] * 4)
        del Y
        o_us, b_us, same = vendor_i32(torch, L, X, W)
        per[name] = dict(us=round(us, 2), tops=round(2.0 * M * n * k / us / 1e6, 1), i32_us=round(o_us, 2),
                         hipblaslt_i32_us=round(b_us, 2), hipblaslt_equal=same)
        total_us += us
        ops += 2.0 * M * n * k
        vend["ours"] += o_us
        vend["blas"] += b_us
        vend["equal"] &= same
        del X, W
        torch.cuda.empty_cache()
    import oracle as O
    ctops, ct, ran, cores = cpu_linears(torch, np, O, 2048, {"o": (4096, 4096)}, budget_s=1.0)
    out = dict(us_per_layer=round(total_us, 1), tops=round(ops / total_us / 1e6, 1),
               frac_of_peak=round(ops / total_us / 1e6 / PEAK_INT8_TOPS, 4), per_linear=per,
               vs_hipblaslt=dict(ours_i32_us_per_layer=round(vend["ours"], 1),
                                 hipblaslt_i32_us_per_layer=round(vend["blas"], 1), outputs_equal=vend["equal"],
                                 note="the same int8 operands, int32 out: uwc_igemm_i32 against torch._int_mm "
                                      "(hipBLASLt), graph-replayed on this box"),
               cpu_baseline=dict(value=round(ctops, 4), unit="TOPS", cores=cores, kind="port", **host_cpu(),
                                 sample=f"quant_act + fp64 matmul + dequant of the o linear at M=2048 "
                                        f"(a quarter of the prefill rows), {ct:.2f} s"))
    log(f"llama prefill: {out}")
    return out


QWEN3_1P7B = dict(D=2048, H=16, Hkv=8, hd=128, I=6144, L=28, V=151936, eps=1e-6, Bs=512, max_pos=8192, theta=1e6,
                  arch=0)


def _oracle_model(m, layers, token_rows):
    """The oracle's Model for the first `layers` layers of a GPU DetModel, with the embedding
    restricted to token_rows (the tokens are remapped to 0 .. len - 1)."""
    import numpy as np
    from oracle import detrt_stage as S
    c = lambda t: t.detach().cpu().numpy()  # noqa: E731
    cfg = dict(QWEN3_1P7B, eps_bits=int(np.float32(QWEN3_1P7B["eps"]).view(np.uint32)))
    norms = [{nm: c(L[nm]) for nm in ("in_norm", "post_norm", "q_norm", "k_norm")} for L in m.layers[:layers]]
    lins = [{nm: (c(L[nm].Wq), c(L[nm].sw)) for nm in ("qkv", "o", "gu", "down")} for L in m.layers[:layers]]
    emb = c(m.embed[token_rows])
    om = S.Model(cfg, emb, norms, lins, c(m.cos), c(m.sin), lm_head=(c(m.lm_head.Wq), c(m.lm_head.sw)),
                 final_norm=c(m.norm))
    return om


def qwen3_e2e(args, torch, np):
    """the deterministic Qwen3-1.7B-shaped integer forward (28 layers, vocab
    151936, seeded random weights quantized per detrt on the GPU) over one 8192-token prompt of
    seeded uniform ids: embedding, 28 fused decoder layers (rmsnorm_quant, qkv GEMM, qkv_post,
    exact attention, o GEMM + residual, rmsnorm_quant, gate_up GEMM, swiglu_quant, down GEMM +
    residual), every layer's stage-output root (SHA-256 Merkle over its 8192 output rows) on the
    GPU, then the final norm, the lm_head GEMM (int32 logits) and a SHA-256 Merkle root of the
    logits rows. Parity: the same model's first two layers and the lm_head at T = 64 against the
    CPU oracle, bit for bit (outputs, stage roots, int logits)."""
    from uwc_amd import detgpu
    from oracle import detrt_stage as S
    cfg = QWEN3_1P7B
    T, NL = args.e2e_tokens, args.e2e_layers
    cfg = dict(cfg, L=NL)
    dev = "cuda"
    t0 = time.perf_counter()
    m = detgpu.DetModel.random(cfg, seed=5, device=dev)
    torch.cuda.synchronize()
    log(f"e2e: model of {NL} layers built in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(2026)
    toks = rng.integers(0, cfg["V"], size=T)
    tokens = torch.from_numpy(toks[None]).to(dev)

    louts = torch.empty((NL, T, cfg["D"]), dtype=torch.float32, device=dev)  # every layer's output

    def forward(tok):
        x, roots = detgpu.forward_stage_roots(m, tok, outs=louts)
        acc, _ = detgpu.final_logits(m, x)
        lroot = detgpu.merkle_roots(detgpu._row_leaf_words(acc, detgpu.TAG_SOUT, 0, 0), 1)
        return x, roots, acc, lroot

    forward(tokens)  # warm-up
    torch.cuda.synchronize()
    reps = 2
    t0 = time.perf_counter()
    for _ in range(reps):
        x, roots, acc, lroot = forward(tokens)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    D, H, Hkv, hd, I, V = cfg["D"], cfg["H"], cfg["Hkv"], cfg["hd"], cfg["I"], cfg["V"]
    lin_macs = T * D * ((H + 2 * Hkv) * hd + H * hd + 2 * I) + T * I * D
    gemm_ops = 2.0 * (NL * lin_macs + T * D * V)
    attn_macs = NL * H * hd * T * (T + 1) // 2 * 2  # q.k and p.v over the causal half
    layer_roots = detgpu.digest_bytes(roots)
    import hashlib
    out = dict(workload=f"Qwen3-1.7B-shaped deterministic integer forward, {NL} layers, vocab {V}, {T} tokens, "
                        "random-init weights quantized per detrt; per-layer stage-output roots and the int32 "
                        "logits' Merkle root on the GPU",
               ms_per_forward=round(dt * 1e3, 2), tokens_per_s=round(T / dt, 1),
               gemm_tops=round(gemm_ops / dt / 1e12, 1),
               attention_gmac=round(attn_macs / 1e9, 1),
               layer_roots_sha256=hashlib.sha256(b"".join(bytes(r) for r in layer_roots)).hexdigest()[:20],
               first_layer_root=bytes(layer_roots[0]).hex()[:20],
               logits_root=bytes(detgpu.digest_bytes(lroot)[0]).hex()[:20])
    log(f"e2e: {out}")
    del x, roots, acc, lroot, louts
    torch.cuda.empty_cache()
    # parity at T = 64: two layers + lm_head vs the oracle
    Tp = 64
    sub = toks[:Tp]
    uniq, inv = np.unique(sub, return_inverse=True)
    om = _oracle_model(m, 2, torch.from_numpy(uniq).to(dev))
    tk = torch.from_numpy(sub[None]).to(dev)
    xg = detgpu.embed(m.embed, tk)
    xo = om.embed[inv]
    ok_rows, ok_roots = True, True
    for l in range(2):
        xg = detgpu.layer_fused(m, m.layers[l], xg, 1, Tp)
        xo = S.layer(om, l, xo)
        ok_rows &= bool(np.array_equal(xg.cpu().numpy().view(np.uint32), xo.view(np.uint32)))
        ok_roots &= detgpu.stage_output_roots(xg.reshape(1, Tp, D))[0] == S.stage_output_root(xo)
    acc_g, _ = detgpu.final_logits(m, xg)
    acc_o, _ = S.final_logits(om, xo)
    out["parity"] = dict(tokens=Tp, layers=2, outputs_equal=ok_rows, stage_roots_equal=ok_roots,
                         int_logits_equal=bool(np.array_equal(acc_g.cpu().numpy(), acc_o)))
    # CPU baseline: the oracle's layer at Tc tokens (float64 BLAS GEMMs as the reference's CPU path)
    Tc = args.e2e_cpu_tokens
    subc = toks[:Tc]
    uc, ic = np.unique(subc, return_inverse=True)
    omc = _oracle_model(m, 1, torch.from_numpy(uc).to(dev))
    threads = os.cpu_count() or 1
    t0 = time.perf_counter()
    S.layer(omc, 0, omc.embed[ic])
    ct = time.perf_counter() - t0
    cl_ops = 2.0 * Tc * D * ((H + 2 * Hkv) * hd + H * hd + 2 * I) + 2.0 * Tc * I * D
    out["cpu_baseline"] = dict(value=round(cl_ops / ct / 1e12, 5), unit="TOPS (linear ops / whole-layer time)",
                               cores=threads, kind="port", **host_cpu(),
                               sample=f"one decoder layer at T={Tc} through oracle/detrt_stage.py (numpy fp32 "
                                      f"ops, float64 BLAS GEMMs), {ct:.2f} s")
    out["gemm_tops_unit"] = "TOPS (linear + lm_head ops / whole-forward time)"
    log(f"e2e parity / cpu: {out['parity']} {out['cpu_baseline']}")
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "noisy_gemm256_mining_4096_traffic.txt")
COPY_BYTES = 256 << 20  # the calibration copy: reads and writes exactly this many bytes


def traffic_probe(args, torch, ops, O, np):
    """What the two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE) profile: a few mined
    forwards at the bench shape (one group: batched GEMM launches of args.gemm_group nonces),
    then a plain device copy of COPY_BYTES three times, whose counter readings calibrate the KiB
    units of both counters."""
    args.steps, args.warmup, args.warmup_seconds = args.gemm_group, args.gemm_group, 0.0
    mining(args, torch, np, ops)
    x = torch.empty(COPY_BYTES, dtype=torch.int8, device="cuda").fill_(1)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    log("traffic probe: done")


def linear_traffic_cases():
    """The kernels whose HBM traffic --linears-traffic-probe measures, in order: (case name, m, n, k,
    what, algorithmic bytes). what: "gemm" = exact GEMM with the fused fp32 dequant
    (uwc_igemm_dequant_f32: X int8 m x k, W int8 n x k, fp32 out and scales), "quant" = quant_act of
    an fp32 m x k input (bs 512: int8 out and one scale per row)."""
    cases = [("configs[0] mlp_up", 64, 6144, 2048, "gemm")]
    for m in (1, 8, 32):
        cases += [(f"decode M={m} {nm}", m, n, k, "gemm") for nm, (n, k) in LLAMA_LINEARS.items()]
    cases += [("configs[1] quant_act 2048x2048", 2048, 0, 2048, "quant"),
              ("configs[1] quant_act 2048x6144", 2048, 0, 6144, "quant")]
    cases += [(f"configs[1] {nm}", 2048, n, k, "gemm") for nm, (n, k) in
              (("qkv", (4096, 2048)), ("o", (2048, 2048)), ("gu", (12288, 2048)), ("down", (2048, 6144)))]
    out = []
    for name, m, n, k, what in cases:
        byt = (n * k + m * k + 4 * m * n + 4 * (m + n)) if what == "gemm" else (m * k * 5 + 4 * m)
        out.append((name, m, n, k, what, byt))
    return out


ATTN_FILE = os.path.join(ROOT, "profiles", "attention_8192_counters.txt")
ATTN_SHAPE = (8192, 16, 8, 128)  # configs[4]'s attention: T, heads, kv heads, head_dim (Qwen3-1.7B)
ATTN_REPS = 4


def attention_probe(torch):
    """What the attention profile's passes run: configs[4]'s attention in the stored-exponentials
    form (v_transpose_kernel, attn_rowmax_kernel, then attention_kernel<128, true>) ATTN_REPS times
    on random int8 heads, then the calibration copy of COPY_BYTES three times."""
    from uwc_amd import detgpu
    T, H, Hkv, hd = ATTN_SHAPE
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    qq = torch.randint(-127, 128, (T, H, hd), dtype=torch.int8, device=dev, generator=g)
    kq = torch.randint(-127, 128, (T, Hkv, hd), dtype=torch.int8, device=dev, generator=g)
    vq = torch.randint(-127, 128, (T, Hkv, hd), dtype=torch.int8, device=dev, generator=g)
    qs, ks, vs = (torch.rand((T, h, 1), device=dev, generator=g) * 3e-2 + 1e-3 for h in (H, Hkv, Hkv))
    for _ in range(ATTN_REPS):
        detgpu.attention(qq, qs, kq, ks, vq, vs, 1, T, H, Hkv, float(1.0 / hd ** 0.5), stored_exp=True)
    x = torch.empty(COPY_BYTES, dtype=torch.int8, device=dev).fill_(1)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    log("attention probe: done")


def summarize_attention(stats_csv, sq_csv, fetch_csv, write_csv, cmd):
    """The attention profile from four passes over `bench.py --attention-probe` (a kernel trace
    with --stats, one --pmc pass of SQ counters with GRBM_GUI_ACTIVE, one of FETCH_SIZE, one of
    WRITE_SIZE), per kernel: average duration, VALU instructions per score element, VALU busy,
    the waves' wait share, LDS bank conflicts and HBM bytes (KiB counters scaled by the
    calibration copy), into ATTN_FILE. GRBM_GUI_ACTIVE sums the 8 XCDs' active cycles, so one XCD's
    are a dispatch's cycles; VALU busy = SQ_ACTIVE_INST_VALU x 4 cycles / (1024 SIMDs x one XCD's
    active cycles)."""
    import csv
    import statistics
    T, H, Hkv, hd = ATTN_SHAPE
    scores = H * T * (T + 1) // 2
    kernels = {"attention_kernel<128, true>": "attention_kernel<128, true> (sums, then P x V)",
               "attn_rowmax_kernel<128, 4, 2>": "attn_rowmax_kernel<128, 4, 2> (row maxima)"}

    def per_kernel(path):
        vals = {}
        for row in csv.DictReader(open(path)):
            vals.setdefault((row["Kernel_Name"], row["Counter_Name"]), []).append(float(row["Counter_Value"]))
        return vals

    sq, fetch, write = per_kernel(sq_csv), per_kernel(fetch_csv), per_kernel(write_csv)
    durs = {r["Name"]: float(r["AverageNs"]) for r in csv.DictReader(open(stats_csv))}

    def med(vals, key, counter):
        xs = [x for (n, c), v in vals.items() if key in n and c.startswith(counter) for x in v]
        return statistics.median(xs), len(xs)

    def calib(vals, counter):
        xs = [x for (n, c), v in vals.items() if "copy" in n.lower() and c.startswith(counter) for x in v]
        return COPY_BYTES / (statistics.median([x for x in xs if x > 0.5 * COPY_BYTES / 1024]) * 1024.0)

    ff, wf = calib(fetch, "FETCH_SIZE"), calib(write, "WRITE_SIZE")
    exp_bytes = 4096 * H * sum(wq // 4 + 1 for wq in range(T // 16))
    with open(ATTN_FILE, "w") as f:
        f.write(f"rocprofv3 profile of configs[4]'s attention (Qwen3-1.7B: T = {T}, {H} heads, {Hkv} kv heads, head_dim "
                f"{hd}; stored-exponentials form), medians per dispatch over the probe's {ATTN_REPS} calls\n")
        f.write(f"commands: {cmd}\n")
        f.write(f"score elements per call: {scores} (causal triangle x heads); exponentials stored: {exp_bytes} B, "
                f"written once and read once\n")
        f.write(f"calibration factors: FETCH_SIZE {ff:.4f}, WRITE_SIZE {wf:.4f} (a {COPY_BYTES} B device copy)\n\n")
        for key, label in kernels.items():
            dur = next((v for n, v in durs.items() if key in n), float("nan")) / 1e3
            insts, n = med(sq, key, "SQ_INSTS_VALU")
            act, _ = med(sq, key, "SQ_ACTIVE_INST_VALU")
            gui, _ = med(sq, key, "GRBM_GUI_ACTIVE")
            wcyc, _ = med(sq, key, "SQ_WAVE_CYCLES")
            wait, _ = med(sq, key, "SQ_WAIT_INST_ANY")
            lds, _ = med(sq, key, "SQ_INSTS_LDS")
            bank, _ = med(sq, key, "SQ_LDS_BANK_CONFLICT")
            fb = med(fetch, key, "FETCH_SIZE")[0] * 1024.0 * ff
            wb = med(write, key, "WRITE_SIZE")[0] * 1024.0 * wf
            f.write(f"{label}\n")
            f.write(f"  average duration: {dur:.1f} us (kernel trace); dispatches counted: {n}\n")
            f.write(f"  VALU wave-instructions: {insts:.0f} = {insts * 64 / scores:.1f} per score element\n")
            f.write(f"  VALU busy: {4 * act / (1024 * gui / 8):.3f}; waves waiting on an instruction's inputs: "
                    f"{wait / wcyc:.3f} of their cycles\n")
            f.write(f"  LDS instructions: {lds:.0f}; LDS bank conflict cycles: {bank:.0f}\n")
            f.write(f"  HBM: read {fb / 1e9:.3f} GB, written {wb / 1e9:.3f} GB = {(fb + wb) / 1e9:.3f} GB, "
                    f"{(fb + wb) / (dur * 1e-6) / 1e12:.2f} TB/s over the average duration\n\n")
    print(open(ATTN_FILE).read())


LT_REPS = 3


def linears_traffic_probe(torch):
    """What the rocprofv3 --pmc passes over the linears profile: every case of linear_traffic_cases()
    LT_REPS times (a distinct weight buffer each time), each case preceded by one tiny
    mfma_rate_kernel dispatch that marks where it starts, then the calibration copy."""
    from uwc_amd import _lib, detrt
    dev = "cuda"
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    sink = torch.zeros(1 << 20, dtype=torch.int32, device=dev)
    for name, m, n, k, what, _ in linear_traffic_cases():
        if what == "gemm":
            Ws = [torch.randint(-64, 65, (n, k), dtype=torch.int8, device=dev) for _ in range(LT_REPS)]
            X = torch.randint(-64, 65, (m, k), dtype=torch.int8, device=dev)
            sx, sw = torch.rand(m, device=dev) + 0.5, torch.rand(n, device=dev) * 1e-3
            Y = torch.empty((m, n), dtype=torch.float32, device=dev)
        else:
            xs = [torch.randn((m, k), device=dev) for _ in range(LT_REPS)]
        torch.cuda.synchronize()
        _lib.call("uwc_mfma_rate_probe", 1, 0, sink.data_ptr(), sink.numel(), st())  # the case marker
        for i in range(LT_REPS):
            if what == "gemm":
                _lib.call("uwc_igemm_dequant_f32", X.data_ptr(), Ws[i].data_ptr(), m, n, k, sx.data_ptr(),
                          sw.data_ptr(), Y.data_ptr(), st())
            else:
                detrt.quant_act(xs[i], 512)
        torch.cuda.synchronize()
        log(f"linears traffic probe: {name}")
    x = torch.empty(COPY_BYTES, dtype=torch.int8, device=dev).fill_(1)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    _lib.call("uwc_mfma_rate_probe", 1, 0, sink.data_ptr(), sink.numel(), st())
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    log("linears traffic probe: done")


def summarize_linears_traffic(fetch_csv, write_csv, out_path, cmd):
    """FETCH_SIZE / WRITE_SIZE per dispatch of every case of linears_traffic_probe, calibrated by the
    256 MiB copy, against the case's algorithmic bytes, into out_path."""
    import csv
    import statistics

    def segments(path, counter):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"].startswith(counter)]
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        segs, cur = [], None
        for r in rows:
            if "mfma_rate_kernel" in r["Kernel_Name"]:
                cur = []
                segs.append(cur)
            elif cur is not None and not r["Kernel_Name"].startswith("void at::"):
                # torch's own kernels are the next case's tensor set-up, not this case's work
                cur.append((r["Kernel_Name"].replace("(anonymous namespace)::", ""), float(r["Counter_Value"])))
        return segs

    cases = linear_traffic_cases()
    res = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        segs = segments(path, counter)
        assert len(segs) == len(cases) + 1, f"{counter}: {len(segs)} marked segments for {len(cases)} cases + copy"
        copy = [v for nm, v in segs[-1] if "copy" in nm.lower() and v > 0.5 * COPY_BYTES / 1024]
        assert copy, f"{counter}: no calibration copy after the last marker"
        factor = COPY_BYTES / (statistics.median(copy) * 1024.0)
        for c, seg in zip(cases, segs[:-1]):
            per = {}
            for nm, v in seg:
                per.setdefault(nm.split("(")[0], []).append(v)
            res.setdefault(c[0], {})[counter] = (factor, {nm: statistics.median(vs) * 1024.0 * factor
                                                          for nm, vs in per.items()})
    with open(out_path, "w") as f:
        f.write("HBM traffic (rocprofv3 FETCH_SIZE, WRITE_SIZE) of the configs[0], decode and configs[1] kernels, "
                f"median per dispatch over {LT_REPS} (distinct weight buffers), calibrated by a {COPY_BYTES} B copy\n")
        f.write(f"commands: {cmd}\n")
        f.write(f"calibration factors: FETCH_SIZE {res[cases[0][0]]['FETCH_SIZE'][0]:.4f}, WRITE_SIZE "
                f"{res[cases[0][0]]['WRITE_SIZE'][0]:.4f}\n\n")
        f.write(f"{'case':34s} {'kernel':44s} {'read MB':>9s} {'write MB':>9s} {'total MB':>9s} {'algo MB':>9s} {'ratio':>6s}\n")
        for name, m, n, k, what, byt in cases:
            fr, wr = res[name]["FETCH_SIZE"][1], res[name]["WRITE_SIZE"][1]
            for kn in sorted(set(fr) | set(wr)):
                rd, wt = fr.get(kn, 0.0), wr.get(kn, 0.0)
                f.write(f"{name:34s} {kn[:44]:44s} {rd / 1e6:9.2f} {wt / 1e6:9.2f} {(rd + wt) / 1e6:9.2f} "
                        f"{byt / 1e6:9.2f} {(rd + wt) / byt:6.2f}\n")
        f.write("\nalgo MB: W + X + fp32 out + scales for the GEMMs (uwc_igemm_dequant_f32); fp32 in + int8 out + "
                "scales for quant_act. ratio > 1: bytes fetched or written beyond the algorithmic ones (e.g. the "
                "skinny kernels' X broadcast to every workgroup, or W rows read twice through L2).\n")
    print(open(out_path).read())


def summarize_pmc(fetch_csv, write_csv, cmd, nonces):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE of the noisy GEMM, each scaled by COPY_BYTES over the
    counter's reading for the calibration copy, into TRAFFIC_FILE."""
    import csv
    import statistics

    def per_kernel(path, counter):
        vals = {}
        for row in csv.DictReader(open(path)):
            if row["Counter_Name"].startswith(counter):
                vals.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return vals

    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        v = per_kernel(path, counter)
        gemm = [x for name, xs in v.items() if "noisy_gemm256_kernel<true, true, 1, true>" in name for x in xs]
        copy = [x for name, xs in v.items() if "copy" in name.lower() for x in xs]  # the runtime's blit kernel
        copy = [x for x in copy if x > 0.5 * COPY_BYTES / 1024]  # the 256 MiB copies, not tensor setup
        gk, ck = statistics.median(gemm), statistics.median(copy)
        factor = COPY_BYTES / (ck * 1024.0)
        out[counter] = dict(gemm_kib=gk, copy_kib=ck, factor=factor, bytes=gk * 1024.0 * factor, n=len(gemm))
    traffic = out["FETCH_SIZE"]["bytes"] + out["WRITE_SIZE"]["bytes"]
    nonces = int(nonces)
    with open(TRAFFIC_FILE, "w") as f:
        f.write(f"HBM traffic of noisy_gemm256_kernel<true, true, 1, true> (mining, 4096^3, r=64, L=2), bytes per dispatch "
                f"of {nonces} nonces\n")
        f.write(f"commands: {cmd}\n")
        for c in ("FETCH_SIZE", "WRITE_SIZE"):
            d = out[c]
            f.write(f"{c}: median {d['gemm_kib']:.1f} KiB per dispatch over {d['n']} dispatches; calibration copy of "
                    f"{COPY_BYTES} B reads {d['copy_kib']:.1f} KiB -> factor {d['factor']:.4f} -> {d['bytes']:.0f} B\n")
        f.write(f"traffic_bytes_per_launch: {traffic:.0f}\n")
        f.write(f"traffic_bytes_per_nonce: {traffic / nonces:.0f} (read {out['FETCH_SIZE']['bytes'] / nonces:.0f}, "
                f"written {out['WRITE_SIZE']['bytes'] / nonces:.0f}; algorithmic: A 16.8 MB + B 16.8 MB + corrections "
                f"2.1 MB read, int32 output 67.1 MB written)\n")
    print(open(TRAFFIC_FILE).read())


def summarize_counters(csv_path, cmd, nonces):
    """Per-dispatch counters of the hashed GEMM (median over its dispatches) from one rocprofv3 --pmc
    pass over `bench.py --traffic-probe`, into COUNTER_FILE, with the matrix-core busy fraction.
    SQ_VALU_MFMA_BUSY_CYCLES sums, over every SIMD, the cycles its matrix core works (it equals the
    dispatch's MFMA work: 8 nonces x 73.0 GMAC / 1024 MAC per cycle); GRBM_GUI_ACTIVE sums the
    active cycles of the 8 XCDs' graphics blocks. busy fraction = MFMA cycles / (active cycles of
    one XCD x 1024 SIMDs)."""
    import csv
    import statistics
    vals = {}
    for row in csv.DictReader(open(csv_path)):
        if "noisy_gemm256_kernel<true, true, 1, true>" in row["Kernel_Name"]:
            vals.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
    med = {c: statistics.median(v) for c, v in vals.items()}
    simds, xcds = 256 * 4, 8
    busy, active = med.get("SQ_VALU_MFMA_BUSY_CYCLES"), med.get("GRBM_GUI_ACTIVE")
    frac = busy / (active / xcds * simds) if busy and active else None
    nonces = int(nonces)
    with open(COUNTER_FILE, "w") as f:
        f.write(f"rocprofv3 counters of noisy_gemm256_kernel<true, true, 1, true> (mining 4096^3, r=64, {nonces} nonces "
                f"per dispatch), median per dispatch over {len(next(iter(vals.values())))} dispatches\n")
        f.write(f"command: {cmd}\n")
        for c in sorted(med):
            f.write(f"{c}: {med[c]:.0f}\n")
        if frac is not None:
            f.write(f"mfma_busy_frac: {frac:.4f} (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {xcds} XCDs x {simds} "
                    f"SIMDs))\n")
            f.write(f"active_cycles_per_xcd: {active / xcds:.0f} (divide by the dispatch's duration for the clock)\n")
        if "SQ_INSTS_VALU_MFMA_MOPS_I8" in med and active:
            f.write(f"mfma_i8_ops_per_dispatch: {med['SQ_INSTS_VALU_MFMA_MOPS_I8'] * 512:.4g} "
                    "(SQ_INSTS_VALU_MFMA_MOPS_I8 x 512)\n")
    print(open(COUNTER_FILE).read())


def summarize_side_counters(sq_csv, fetch_csv, write_csv, out_path, cmd, nonces):
    """Per-dispatch counters (median over the dispatches) of the sweep's operand-side and
    commitment kernels from three rocprofv3 --pmc passes over `bench.py --traffic-probe` (SQ
    counters, then FETCH_SIZE, then WRITE_SIZE; the byte counters scaled by what they read for the
    calibration copy of COPY_BYTES), with the VALU busy fraction (wave-instructions x 4 cycles over
    the SIMDs' active cycles) and the fraction of wave cycles spent waiting."""
    import csv
    import statistics
    kernels = ("side_many_kernel<4>", "b3_lanes_kernel")

    def per_dispatch(path):
        d = {}
        for row in csv.DictReader(open(path)):
            key = (row["Dispatch_Id"], row["Kernel_Name"])
            d.setdefault(key, {})
            d[key][row["Counter_Name"]] = d[key].get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
        return d

    def medians(d, pat):
        rows = [c for (_, kn), c in d.items() if pat in kn]
        return {c: statistics.median(r.get(c, 0.0) for r in rows) for c in rows[0]} if rows else {}, len(rows)

    byte_factor = {}
    for ctr, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        d = per_dispatch(path)
        copies = [c[ctr] for (_, kn), c in d.items() if "copy" in kn.lower() and c.get(ctr, 0) > 0.5 * COPY_BYTES / 1024]
        byte_factor[ctr] = (d, COPY_BYTES / (statistics.median(copies) * 1024.0))
    sq = per_dispatch(sq_csv)
    simds, xcds, nonces = 256 * 4, 8, int(nonces)
    with open(out_path, "w") as f:
        f.write(f"rocprofv3 counters of the mining sweep's operand side and commitment (4096^3, r=64, {nonces} nonces "
                "per dispatch), median per dispatch\n")
        f.write(f"commands: {cmd}\n")
        for kname in kernels:
            med, n = medians(sq, kname)
            if not med:
                continue
            f.write(f"\n{kname} ({n} dispatches)\n")
            for c in sorted(med):
                f.write(f"  {c}: {med[c]:.0f}\n")
            active = med.get("GRBM_GUI_ACTIVE", 0.0) / xcds
            if active and "SQ_INSTS_VALU" in med:
                f.write(f"  valu_busy_frac: {med['SQ_INSTS_VALU'] * 4 / (active * simds):.3f} (SQ_INSTS_VALU x 4 / "
                        f"(GRBM_GUI_ACTIVE / {xcds} x {simds}))\n")
            if med.get("SQ_WAVE_CYCLES"):
                f.write(f"  wait_any_frac: {med.get('SQ_WAIT_ANY', 0) / med['SQ_WAVE_CYCLES']:.3f}, wait_inst_any_frac: "
                        f"{med.get('SQ_WAIT_INST_ANY', 0) / med['SQ_WAVE_CYCLES']:.3f} (of SQ_WAVE_CYCLES)\n")
            for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
                d, fac = byte_factor[ctr]
                bm, _ = medians(d, kname)
                if ctr in bm:
                    f.write(f"  {ctr}: {bm[ctr]:.0f} KiB x {fac:.4f} = {bm[ctr] * 1024 * fac / 1e6:.1f} MB per dispatch, "
                            f"{bm[ctr] * 1024 * fac / 1e6 / nonces:.2f} MB per nonce\n")
    print(open(out_path).read())


def gemm_reps(steps: int) -> int:
    """Back-to-back launches of the noisy GEMM that time it after the sweep."""
    return max(8, min(steps, 64))


def summarize_trace(trace_csv, out_path, cmd, steps, warmup, group):
    """A kernel trace (run_kernel_trace.csv) of `bench.py --no-cpu --no-detrt --no-e2e --steps S
    --warmup W ...` (groups of G nonces, one batched GEMM launch per group) as text: per kernel of
    the timed sweep (from the end of the warm-up's last GEMM launch to the end of the sweep's last)
    calls, average and time per nonce, and the average of the back-to-back GEMM launches that give
    the bench's roofline figure. The warm-up runs for a time, so the sweep is found from the end:
    its S / G GEMM launches are followed by the capture call's launch, two untimed launches and the
    timed back-to-back ones."""
    import csv
    import re
    steps, warmup, group = int(steps), int(warmup), int(group)
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    name = lambda r: re.sub(r"\(.*", "", r["Kernel_Name"])  # noqa: E731
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # noqa: E731
    g = [i for i, r in enumerate(rows) if "noisy_gemm256_kernel<true, true, 1, true>" in r["Kernel_Name"]]
    ns, nb = -(-steps // group), gemm_reps(steps)  # GEMM launches of the sweep, timed back-to-back launches
    first = len(g) - nb - 3 - ns  # index in g of the sweep's first GEMM launch
    assert first >= 1, "trace too short for a warm-up, a sweep and the back-to-back launches"
    t0, t1 = int(rows[g[first - 1]]["End_Timestamp"]), int(rows[g[first + ns - 1]]["End_Timestamp"])
    per = {}
    for r in rows:
        if t0 < int(r["Start_Timestamp"]) and int(r["End_Timestamp"]) <= t1:
            per.setdefault(name(r), []).append(dur(r))
    b2b = [dur(rows[i]) for i in g[len(g) - nb:]]
    with open(out_path, "w") as f:
        f.write(f"rocprofv3 kernel trace, mined forward 4096x4096x4096 r=64 (bench.py workload), sweep of {steps} "
                f"nonces after {first * group} warm-up nonces, {group} nonces per group\n")
        f.write(f"command: {cmd}\n\n")
        f.write(f"timed sweep: {(t1 - t0) / 1e3 / steps:.2f} us per nonce (kernel trace clock)\n")
        f.write(f"{'kernel':58s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'us/nonce':>9s}\n")
        for k_, xs in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            f.write(f"{k_[:58]:58s} {len(xs):6d} {sum(xs) / len(xs):9.2f} {min(xs):9.2f} {max(xs):9.2f} "
                    f"{sum(xs) / steps:9.2f}\n")
        f.write(f"\nback-to-back noisy_gemm256_kernel<true, true, 1, true> launches of {group} nonces (the bench's "
                f"roofline figure): {len(b2b)} calls, avg {sum(b2b) / len(b2b):.2f} us = "
                f"{sum(b2b) / len(b2b) / group:.2f} us per nonce, min {min(b2b):.2f}, max {max(b2b):.2f}\n")
        f.write(f"\nPer group of {group} nonces: b3_lanes (or, below 4 operands, b3_chunks) + b3_reduce (one batched "
                "commitment of the group's A) and\n"
                "one nonce_noise (E_A, P_A, selection matrices of the group), on a side stream one group ahead, beside\n"
                "the previous group's side work; one side_many_kernel launch (noised A and both projections in limbs\n"
                "for every nonce of the group);\n"
                "one noisy_gemm256_kernel<true, true, 1, true> launch (the group's hashed GEMMs with exact denoise,\n"
                "int32 out; split roles, stores overlapping the next nonce). Kernel times overlap: per-nonce sums\n"
                "exceed the sweep's wall time per nonce.\n")
    print(open(out_path).read())


def summarize_e2e_trace(stats_csv, out_path, cmd):
    """The kernel-trace --stats table of a `bench.py --e2e-only` run as text: per kernel
    calls, average and share, plus per-forward totals (3 forwards: one warm-up, two timed)."""
    import csv
    import re
    rows = list(csv.DictReader(open(stats_csv)))
    with open(out_path, "w") as f:
        f.write("rocprofv3 kernel trace, configs[4]: 28-layer Qwen3-1.7B-shaped integer forward over 8192 tokens "
                "(bench.py --e2e-only: 3 forwards + the T=64 parity run and the CPU-baseline weight copies)\n")
        f.write(f"command: {cmd}\n\n")
        f.write(f"{'kernel':58s} {'calls':>6s} {'avg_us':>9s} {'ms/fwd':>8s} {'share':>6s}\n")
        for r in rows:
            name = re.sub(r"\(.*", "", r["Name"].replace("(anonymous namespace)::", ""))[:58]
            f.write(f"{name:58s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:9.2f} "
                    f"{float(r['TotalDurationNs']) / 3e6:8.2f} {float(r['Percentage']):5.1f}%\n")
        f.write("\nPer forward: 28 x (rmsnorm_quant_wave_kernel x 2, noisy_gemm256_kernel<false, false, 1, true> "
                "(the persistent multi-tile form) for qkv and gate_up, noisy_gemm256_kernel<false, false, 4, false> for "
                "o and down (dequant and residual add in the epilogue), qkv_post_kernel, the stored-exponentials "
                "attention in two launches (attn_rowmax_kernel: the row maxima; attention_kernel<128, true>: the "
                "exact sums with the exponentials stored, then P x V from them), quant_act_dgroup_kernel, "
                "swiglu_quant_wave_kernel), then one batched set of sha_* launches for all 28 layers' stage-output "
                "roots (sha_block_leaves, sha_row_leaf_quad, sha_group, sha_tree), rmsnorm_quant + the lm_head GEMM "
                "(256x256 tiles + a 128-wide column tail) + its fp32 dequant (dequant4_kernel) + the logits' Merkle root "
                "(sha_block_leaves, sha_row_tree, sha_group, sha_tree); ms/fwd = total / 3 (the buffer copies and "
                "the random-number and scaling kernels are model set-up and the oracle's weight copies, outside the "
                "timed forwards; the T = 64 parity run adds the few small-shape kernels).\n")
    print(open(out_path).read())


LINEAR_LABELS = ["configs[1] layer graph: 4 x (quant_act + GEMM)", "configs[1] qkv GEMM 2048x4096x2048",
                 "configs[1] o GEMM 2048x2048x2048", "configs[1] gu GEMM 2048x12288x2048",
                 "configs[1] down GEMM 2048x2048x6144", "configs[0] mlp_up 64x6144x2048"] + [
    f"Llama-3.1-8B decode M={m} {nm}" for m in (1, 8, 32) for nm in ("qkv 6144x4096", "o 4096x4096",
                                                                      "gu 28672x4096", "down 4096x14336")]


def summarize_linears_trace(trace_csv, out_path, cmd):
    """A kernel trace of `bench.py --linears-only` as text: per graph-timed shape (configs[1]'s layer
    graph and its four GEMMs, configs[0], the Llama-3.1-8B decode linears) the device durations of
    its timed replays. Each graph of N launches is run eagerly, replayed once, then replayed three
    times back to back (N from the bench's own launch counts); a shape whose timed replays are not
    found is left out of the table."""
    import csv
    import re
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    ours = lambda r: not re.search(r"at::native|__amd_rocclr", r["Kernel_Name"])  # noqa: E731
    # configs[1]'s graphs: runs of this library's dispatches split at idle gaps; a shape's timed run
    # is 3 x the launches of its graph, right after the first replay's run of a third of that
    runs, cur, last_end = [], [], None
    for r in rows:
        st, en = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        if cur and (st - last_end > 30000 or not ours(r)):
            runs.append(cur)
            cur = []
        if ours(r):
            cur.append(r)
        last_end = en
    if cur:
        runs.append(cur)
    timed, j = [], 1
    for w in [24] * 5:
        while j < len(runs) and not (len(runs[j]) == w and len(runs[j - 1]) == w // 3):
            j += 1
        timed.append(runs[j] if j < len(runs) else None)
        j += 1
    # the skinny shapes: each rotates N launches over its weights; torch's own kernels (the input's
    # set-up) bracket the eager run, and then the first replay and the three timed ones (4 N launches
    # with no torch kernel among them, however the profiler's stalls split them in time)
    segs, cur = [], []
    for r in rows[rows.index(timed[-1][-1]) + 1 if timed[-1] else 0:]:
        if ours(r):
            cur.append(r)
        elif cur:
            segs.append(cur)
            cur = []
    if cur:
        segs.append(cur)
    j = 0
    for n in [_skinny_launches(6144 * 2048)] + [
            _skinny_launches(nn * kk) for _ in (1, 8, 32) for nn, kk in LLAMA_LINEARS.values()]:
        while j < len(segs) and len(segs[j]) != 4 * n:
            j += 1
        timed.append(segs[j][n:] if j < len(segs) else None)
        j += 1
    with open(out_path, "w") as f:
        f.write("rocprofv3 kernel trace, graph-timed linears of bench.py (configs[1] at M=2048, configs[0], "
                "Llama-3.1-8B decode at M=1, 8, 32; weights rotated over > 1.2 GB)\n")
        f.write(f"command: {cmd}\n\n")
        f.write(f"{'shape':44s} {'kernel':44s} {'grid':>6s} {'lds':>7s} {'calls':>6s} {'avg_us':>8s} {'min_us':>8s} "
                f"{'max_us':>8s}\n")
        for lab, run in zip(LINEAR_LABELS, timed):
            if run is None:
                continue
            per = {}
            for r in run:
                name = r["Kernel_Name"].replace("(anonymous namespace)::", "")
                key = (re.sub(r"\(.*", "", name)[:44], r.get("Grid_Size_X", ""), r.get("LDS_Block_Size", ""))
                per.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            for (kn, grid, lds), xs in per.items():
                f.write(f"{lab[:44]:44s} {kn:44s} {grid:>6s} {lds:>7s} {len(xs):6d} {sum(xs) / len(xs):8.2f} "
                        f"{min(xs):8.2f} {max(xs):8.2f}\n")
        f.write("\ngrid = work-items (workgroups x 640 for skinny_dma_kernel); kernel durations exclude the "
                "~1.8 us launch gap between dependent graph nodes that the bench's per-launch figures include.\n")
    print(open(out_path).read())


def _summary_value(path, key):
    """The number after `key:` in a committed rocprofv3 summary under profiles/, or None."""
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def read_traffic(nonces_per_launch):
    """HBM bytes of one launch of nonces_per_launch nonces: the committed FETCH_SIZE / WRITE_SIZE
    summary's bytes per nonce times the launch's nonces, or None."""
    v = _summary_value(TRAFFIC_FILE, "traffic_bytes_per_nonce")
    return None if v is None else int(v * nonces_per_launch)


COUNTER_FILE = os.path.join(ROOT, "profiles", "noisy_gemm256_mining_4096_counters.txt")


def read_mfma_busy():
    """The hashed GEMM's matrix-core busy fraction from the committed counter summary:
    SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs), or None."""
    return _summary_value(COUNTER_FILE, "mfma_busy_frac")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="nonces timed")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--warmup-seconds", type=float, default=2.0, help="minimum warm-up time before the timed sweep")
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--rank", type=int, default=64)
    ap.add_argument("--distinct", type=int, default=64, help="distinct resident A matrices cycled over")
    ap.add_argument("--out-buffers", type=int, default=8, help="distinct int32 outputs rotated through the sweep")
    ap.add_argument("--group", type=int, default=None,
                    help="nonces per batched commitment / noise launch (default: forward_many's, equal groups of <= 32)")
    ap.add_argument("--gemm-group", type=int, default=None, help="nonces per batched GEMM launch (default: the group)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-max-nonces", type=int, default=4)
    ap.add_argument("--mine-attempts", type=int, default=16, help="noise_mine attempts at the miner's shape")
    ap.add_argument("--no-mine", action="store_true", help="skip the pure noise-mining leg")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-detrt", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip configs[4] (the 28-layer forward)")
    ap.add_argument("--e2e-only", action="store_true", help="run only configs[4]")
    ap.add_argument("--e2e-tokens", type=int, default=8192)
    ap.add_argument("--e2e-layers", type=int, default=28)
    ap.add_argument("--e2e-cpu-tokens", type=int, default=256)
    ap.add_argument("--traffic-probe", action="store_true", help="the workload of the FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--attention-probe", action="store_true",
                    help="configs[4]'s attention a few times, then the calibration copy (the attention profile's workload)")
    ap.add_argument("--summarize-attention", nargs=5, metavar=("STATS_CSV", "SQ_CSV", "FETCH_CSV", "WRITE_CSV", "CMD"),
                    help="write profiles/attention_8192_counters.txt from the attention probe's passes")
    ap.add_argument("--linears-only", action="store_true", help="run only configs[1], configs[0], the decode and the prefill linears")
    ap.add_argument("--linears-traffic-probe", action="store_true",
                    help="the workload of the FETCH_SIZE / WRITE_SIZE passes over the configs[0], decode and configs[1] kernels")
    ap.add_argument("--summarize-linears-traffic", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "OUT", "CMD"),
                    help="write the HBM-traffic summary of a --linears-traffic-probe pair of counter runs")
    ap.add_argument("--summarize-linears-trace", nargs=3, metavar=("TRACE_CSV", "OUT", "CMD"),
                    help="write the graph-timed linears' kernel-trace summary under profiles/")
    ap.add_argument("--summarize-pmc", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "CMD", "NONCES"),
                    help="write the traffic summary under profiles/ from two counter_collection.csv files")
    ap.add_argument("--summarize-side-counters", nargs=6,
                    metavar=("SQ_CSV", "FETCH_CSV", "WRITE_CSV", "OUT", "CMD", "NONCES"),
                    help="write the operand side's and commitment's counter summary")
    ap.add_argument("--summarize-counters", nargs=3, metavar=("COUNTER_CSV", "CMD", "NONCES"),
                    help="write the hashed GEMM's counter summary under profiles/ from a counter_collection.csv")
    ap.add_argument("--summarize-e2e-trace", nargs=3, metavar=("STATS_CSV", "OUT", "CMD"),
                    help="write a configs[4] kernel-trace summary under profiles/")
    ap.add_argument("--summarize-trace", nargs=6, metavar=("TRACE_CSV", "OUT", "CMD", "STEPS", "WARMUP", "GROUP"),
                    help="write a kernel-trace summary under profiles/ from a run_kernel_trace.csv")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
        return
    if args.summarize_linears_trace:
        summarize_linears_trace(*args.summarize_linears_trace)
        return
    if args.summarize_e2e_trace:
        summarize_e2e_trace(*args.summarize_e2e_trace)
        return
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.summarize_side_counters:
        summarize_side_counters(*args.summarize_side_counters)
        return
    if args.summarize_counters:
        summarize_counters(*args.summarize_counters)
        return
    if args.summarize_linears_traffic:
        summarize_linears_traffic(*args.summarize_linears_traffic)
        return
    if args.summarize_attention:
        summarize_attention(*args.summarize_attention)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the multi-GPU layout "
              "is a design in DESIGN.md, not a measured path", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import oracle as O
    from uwc_amd import ops

    if args.group is None:  # forward_many's own choice for a sweep of args.steps nonces
        args.group = ops.sweep_group(args.steps)
    if args.gemm_group is None:
        args.gemm_group = min(args.group, ops.GEMM_GROUP)
    if args.traffic_probe:
        traffic_probe(args, torch, ops, O, np)
        return
    if args.linears_traffic_probe:
        linears_traffic_probe(torch)
        return
    if args.attention_probe:
        attention_probe(torch)
        return
    if args.e2e_only:
        print(json.dumps(qwen3_e2e(args, torch, np)))
        return
    if args.linears_only:
        print(json.dumps({"detrt_layer": detrt_layer(args, torch, np), "detrt_skinny": skinny_linears(args, torch, np),
                          "llama_prefill": llama_prefill(args, torch, np)}))
        return
    ceiling = mfma_ceiling(torch)
    res = mining(args, torch, np, ops)
    mine = None if args.no_mine else noise_mining(args, torch, np, ops)
    parity, cpu = (None, None) if args.no_cpu else parity_and_cpu(args, res, torch, np, ops, O)
    det = None if args.no_detrt else detrt_layer(args, torch, np)
    skinny = None if args.no_detrt else skinny_linears(args, torch, np)
    prefill = None if args.no_detrt else llama_prefill(args, torch, np)
    e2e = None if (args.no_detrt or args.no_e2e) else qwen3_e2e(args, torch, np)
    m, n, k, r = res["m"], res["n"], res["k"], res["r"]
    line = {
        "metric": METRIC,
        "value": round(res["tops"], 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_nonces_run": getattr(args, "warmup_nonces_run", None),
        "ms_per_step": round(res["dt"] * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "frac_of_peak": round(res["tops"] / PEAK_INT8_TOPS, 4),
        "config": {"workload": f"cuPOW NoisyGEMM mined forward (commit + noise + hashed GEMM + exact denoise, int32 out), "
                               f"{m}x{n}x{k}, r={r}, one nonce per step, {args.steps}-nonce sweep",
                   "m": m, "n": n, "k": k, "r": r, "noise": "reference rules (E in [-32,31], +-1 pairs)"},
        "mfma_sustained_tops": ceiling,
        "roofline": {"bound": "mfma", "achieved": round(res["kern_tops"], 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(res["kern_tops"] / PEAK_INT8_TOPS, 4), "traffic": read_traffic(res["per_launch"]),
                     "traffic_source": "profiles/noisy_gemm256_mining_4096_traffic.txt (rocprofv3 FETCH_SIZE + "
                                       "WRITE_SIZE passes over bench.py --traffic-probe, copy-calibrated; bytes per "
                                       "nonce x nonces per launch)",
                     "mfma_busy_frac": read_mfma_busy(),
                     "mfma_busy_source": "profiles/noisy_gemm256_mining_4096_counters.txt (rocprofv3 "
                                         "SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs))",
                     "kernel": "noisy_gemm256_kernel<HASH=true, DENOISE=true, OUT_I32, SPLIT=true>",
                     "avg_us": round(res["launch_ms"] * 1e3, 2), "nonces_per_launch": res["per_launch"],
                     "ops_per_launch": res["per_launch"] * (2 * m * n * k + 2 * m * n * 2 * r * res["L"])},
        "cpu_baseline": cpu,
        "parity": parity,
        "sweep_winners": res["sweep_winners"],
        "noise_mining": mine,
        "detrt_layer": det,
        "detrt_skinny": skinny,
        "llama_prefill": prefill,
        "qwen3_e2e": e2e,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
