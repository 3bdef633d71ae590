"""Benchmark: 48-block Pairformer trunk forward at N=1024 tokens, bf16 compute.

One step = one full PairformerStack forward (48 blocks, c_z=128, c_s=384,
4 triangle heads x 32, tri-mul hidden 128, 16 single heads; 5% random token
padding; synthetic z, s ~ N(0,1), random weights ~ N(0, 0.02), seed 3) with
the HIP triangle kernels, in place (inference form), residual stream z in
float32 and module arithmetic in bf16 (CUDA autocast, the reference's bf16
inference mode).  Inputs are resident in HBM before timing; each step starts
by restoring z from a resident copy (a 512 MB device copy, ~0.1 ms).

Prints ONE JSON line on stdout (progress goes to stderr).  ``value`` is the
trunk's algorithmic throughput in TFLOP/s (flop counts of the path,
multiply-add = 2) over the timed steps, which run without instrumentation.
Per-kernel figures come from one further step during which the library
records HIP events around every launch on the stream it runs on.
``roofline.traffic`` is the dominant kernel's HBM bytes per launch from the
committed rocprofv3 --pmc summary of this workload
(profiles/pmc_traffic_trunk_n<N>.json, made with ``--pmc-probe``), or null.
``cpu_baseline`` times the CPU oracle (fp32) on one block of the same
workload on this host (median of 5).  ``configs`` holds the other workloads
the path is specified on, each timed on the GPU (median of per-iteration HIP
events) and, for the first three and one block of the trunk, on the CPU
oracle (median of 5 runs after 1 warm-up): the N=128 block in fp32, N=384
triangle attention, N=768 triangle multiplication (both directions), one
N=1024 block of the trunk workload in fp32 arithmetic, the N=2048 x 4-block
stress stack with the single track.  ``machine`` holds the MFMA rates and HBM copy
bandwidth measured on this GPU next to the data sheet's.  ``layer_norm``
times the standalone fast LayerNorm (forward and backward) on the workload's
pair tensor shape, N*N x 128 bf16, outside the trunk step.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from opendde_amd import _lib  # noqa: E402
from opendde_amd import workload as wl  # noqa: E402
from opendde_amd.pairformer import PairformerBlock, PairformerStack  # noqa: E402
from opendde_amd.triangular import (TriangleAttention, TriangleMultiplicationIncoming,  # noqa: E402
                                    TriangleMultiplicationOutgoing)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3     # MI355X fp32 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def flops(n, c_z=128, c_s=384, h=4, d=32, ch=128, n_heads=16):
    """Algorithmic flops per launch / per block (same formulas as the oracle's
    accounting; restated here so the product path does not import the oracle)."""
    core = 4.0 * n ** 3 * h * d
    att_lin = 2.0 * n * n * c_z * (5 * h * d + h)
    contract = 2.0 * n ** 3 * ch
    mul_lin = 2.0 * n * n * (4 * c_z * ch + c_z * c_z + ch * c_z)
    trans = 2.0 * n * n * (2 * c_z * 4 * c_z + 4 * c_z * c_z)
    single = (2.0 * n * n * c_z * n_heads + 8.0 * n * c_s * c_s + 4.0 * n * n * c_s
              + 2.0 * n * c_s * c_s + 2.0 * n * (2 * c_s * 4 * c_s + 4 * c_s * c_s))
    block = 2 * (core + att_lin) + 2 * (contract + mul_lin) + trans + (single if c_s else 0)
    single_trans = 2.0 * n * (2 * c_s * 4 * c_s + 4 * c_s * c_s)
    return dict(core=core, att_lin=att_lin, contract=contract, mul_lin=mul_lin, trans=trans,
                single_trans=single_trans, block=block)


def kernel_bytes(n, c_z=128, h=4, ch=128, z_bytes=4, ct_bytes=2):
    """Algorithmic HBM bytes per launch of the memory-bound kernels."""
    jp = (n + 63) // 64 * 64
    np_ = (n + 127) // 128 * 128
    hd = h * 32
    zrw = n * n * c_z * z_bytes
    # q, k, v planes, plus the gate plane off the weight-stationary path (where
    # the output kernel computes the gate from the z rows it reads anyway)
    planes = 3 if (c_z in (64, 128) and hd in (64, 128)) else 4
    return {
        "triatt_proj": zrw + planes * n * jp * hd * ct_bytes + h * jp * jp * 4 + n * jp * 4,
        "triatt_out": n * jp * hd * ct_bytes + 2 * zrw,
        "trimul_proj": zrw + 2 * ch * np_ * np_ * ct_bytes,
        "trimul_out": ch * np_ * np_ * ct_bytes + 2 * zrw,
    }


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def log(msg: str) -> None:
    """Progress line on stderr (stdout carries only the JSON line)."""
    print(msg, file=sys.stderr, flush=True)


def _cpu_params(mod):
    return {k: v.detach().float().cpu() for k, v in mod.named_parameters()}


def cpu_median(fn, runs: int = 5, warm: int = 1):
    """Median wall time (s) of ``runs`` calls of fn after ``warm`` calls."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), ts


def cpu_threads():
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def cpu_baseline(n: int, chunk: int, runs: int = 5):
    """Time the CPU oracle (fp32) on one PairformerBlock of the workload at n:
    a 16-token block first (thread pool and allocator warm-up), then the
    median of ``runs`` runs of the full block."""
    from oracle import reference as ref
    cores = cpu_threads()
    cfg = wl.PairConfig("cpu_sample", n, n_pad=max(0, n * 5 // 100), random_pad=True, seed=3)
    z, s, mask, gen = wl.make_inputs(cfg)
    params = wl.param_values(wl.block_specs(), gen)
    ref.pairformer_block(s[:16], z[:16, :16], mask[:16, :16], params, chunk_size=chunk)
    med, ts = cpu_median(lambda: ref.pairformer_block(s, z, mask, params, chunk_size=chunk),
                         runs=runs, warm=0)
    f = flops(n)["block"]
    return {
        "value": round(f / med / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle (CPU PyTorch restatement of the reference torch path) fp32, one "
                  f"PairformerBlock at N={n} (tri-attn row chunk {chunk}) of the 48, median of "
                  f"{runs} runs ({', '.join(f'{t:.2f}' for t in ts)} s) after a 16-token "
                  f"warm-up; CPU {cpu_model()}, {cores} cores in affinity",
        "block_ms": round(med * 1e3, 1),
    }


def gpu_median_ms(fn, warm: int = 3, iters: int = 20):
    """Median of per-iteration times (HIP events on the current stream, the
    stream every library call here launches on)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(iters)]
    for e0, e1 in evs:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)


def kernel_avg_ms(fn, kid, reps: int = 5):
    """Average launch time of library kernel ``kid`` over ``reps`` calls of
    fn, from the library's HIP events."""
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    tot, cnt = _lib.timing_query(kid)
    _lib.timing_reset()
    return tot / cnt if cnt else None


def probe_machine(dev):
    """Sustained MFMA rates (bf16 16x16x32 on fixed and on pseudo-random
    operands, f32 16x16x4; 2 workgroups of 4 waves per CU, 8 independent
    chains per wave), the attention core's instruction mix as a ceiling
    (odde_probe_mix, also split between the two waves of a SIMD) and HBM bandwidth on this
    GPU: the streaming probe over 2 GiB (read; copy and in-place rewrite,
    bytes read + written) and torch's device copy beside it.  The probes live
    in the measurement library (opendde_amd.probe), not the product library;
    each is timed with events on the stream it launches on."""
    from opendde_amd import probe as pr
    lib = pr.load()
    sink = torch.zeros(256, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    out = {"cus": cus}
    for name, code, iters in (("bf16", pr.BF16, 4000), ("bf16_random", pr.BF16_RANDOM, 4000),
                              ("f32", pr.F32, 1000)):
        fl = ctypes.c_double(0.0)
        call = lambda it: pr.check(lib.odde_probe_mfma(code, it, 2 * cus,  # noqa: E731
                                                       ctypes.c_void_p(sink.data_ptr()),
                                                       ctypes.byref(fl), stream),
                                   "odde_probe_mfma")
        ms = gpu_median_ms(lambda: call(iters), warm=1, iters=3)
        out[f"mfma_{name}_tflops"] = round(fl.value / (ms * 1e-3) / 1e12, 1)
    out["mfma_bf16_tflops_spec"] = PEAK_BF16_TFLOPS
    out["mfma_f32_tflops_spec"] = PEAK_F32_TFLOPS
    # the attention core's per-key-block mix (40 MFMA, 64 exp, 32 bf16 packs)
    # with no memory traffic: its ceiling in attention TF/s on this GPU, and
    # the MFMA and exponential parts alone
    # (split: one wave of each SIMD issues the MFMAs and the other the
    # exponentials and packs -- the most co-issue of the two kinds)
    for name, parts in (("mfma_only", 1), ("exp_only", 2), ("mix", 3), ("split", 4)):
        fl = ctypes.c_double(0.0)
        grid = cus if parts == 4 else 2 * cus  # 8-wave workgroups for the split form
        call = lambda it: pr.check(lib.odde_probe_mix(parts, it, grid,  # noqa: E731
                                                      ctypes.c_void_p(sink.data_ptr()),
                                                      ctypes.byref(fl), stream),
                                   "odde_probe_mix")
        ms = gpu_median_ms(lambda: call(2000), warm=1, iters=3)
        out[f"core_mix_{name}_tflops"] = round(fl.value / (ms * 1e-3) / 1e12, 1)
    src = torch.zeros(1 << 29, device=dev)
    dst = torch.zeros_like(src)
    nbytes = src.numel() * 4
    # the streaming probe (non-temporal loads and stores, as the row-tile
    # kernels stream pair data): read, copy, in-place rewrite
    for name, mode, traffic in (("read", 0, nbytes), ("copy", 1, 2 * nbytes),
                                ("inplace", 2, 2 * nbytes)):
        call = lambda m=mode: pr.check(lib.odde_probe_stream(  # noqa: E731
            m, ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), nbytes, stream),
            "odde_probe_stream")
        ms = gpu_median_ms(call, warm=1, iters=5)
        out[f"hbm_{name}_gbs"] = round(traffic / (ms * 1e-3) / 1e9, 1)
    # torch's device copy of the same 2 GiB, for comparison
    ms = gpu_median_ms(lambda: dst.copy_(src), warm=2, iters=5)
    out["hbm_torch_copy_gbs"] = round(2 * nbytes / (ms * 1e-3) / 1e9, 1)
    out["hbm_gbs_spec"] = PEAK_HBM_GBS
    del src, dst
    torch.cuda.empty_cache()
    return out


def fp32_block_leg(dev, tf32: bool = False):
    """fp32 arithmetic at the trunk's size: one block of the N=1024 workload
    (51 random pads, c_s 384) with fp32 z and no autocast, in place -- the
    reference's default inference precision.  GPU time (median of per-step
    events) and the per-kernel launch times of one further step.  ``tf32``:
    with torch.backends.cuda.matmul.allow_tf32 set, as the reference's
    inference default (enable_tf32) sets it -- the attention core then runs
    its products in three bf16 parts."""
    cfg = wl.TRUNK_N1024
    z, s, mask, gen = wl.make_inputs(cfg)
    blk = PairformerBlock(n_heads=16, c_z=128, c_s=384)
    wl.init_module_(blk, gen)
    blk = blk.eval().to(dev)
    z0, sg, mg = z.to(dev), s.to(dev), mask.to(dev)
    zw = torch.empty_like(z0)

    def fp32_block():
        zw.copy_(z0)
        old = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = tf32
        try:
            with torch.no_grad():
                blk(sg, zw, mg, triangle_multiplicative="hip", triangle_attention="hip",
                    inplace_safe=True)
        finally:
            torch.backends.cuda.matmul.allow_tf32 = old

    ms = gpu_median_ms(fp32_block, warm=2, iters=5)
    f = flops(cfg.n)["block"]
    t = f / (ms * 1e-3) / 1e12
    per_kernel = {}
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    fp32_block()
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    fk = flops(cfg.n)
    for kid, name in _lib.KERNEL_NAMES.items():
        tot, cnt = _lib.timing_query(kid)
        if cnt:
            ent = {"launches": cnt, "avg_ms": round(tot / cnt, 4)}
            fl = {"triatt_core": fk["core"], "trimul_contract": fk["contract"]}.get(name)
            if fl:
                kt = fl / (tot / cnt * 1e-3) / 1e12
                ent.update(tflops=round(kt, 2))
                if tf32:
                    # three bf16 MFMA products per fp32 product: the matrix
                    # pipe executes 3x the algorithmic flops, in bf16
                    ent.update(bf16_mfma_tflops=round(3 * kt, 2),
                               pct_bf16_peak=round(100 * 3 * kt / PEAK_BF16_TFLOPS, 2))
                else:
                    ent.update(pct_f32_peak=round(100 * kt / PEAK_F32_TFLOPS, 2))
            per_kernel[name] = ent
    _lib.timing_reset()
    rate = ({"bf16_mfma_tflops": round(3 * t, 2),
             "pct_bf16_peak": round(100 * 3 * t / PEAK_BF16_TFLOPS, 2)} if tf32 else
            {"pct_f32_peak": round(100 * t / PEAK_F32_TFLOPS, 2)})
    out = dict(
        gpu_ms=round(ms, 3), gflop=round(f / 1e9, 1), tflops=round(t, 2), **rate,
        dtype=("fp32 data; the pair stack's products as three bf16 MFMA parts "
               "(hi*hi + hi*lo + lo*hi, fp32 accumulation)") if tf32 else "fp32",
        residual_dtype="fp32", allow_tf32=tf32, pad_tokens=cfg.n_pad, kernels=per_kernel)
    log(f"bench: fp32 block n=1024{' (tf32 allowed)' if tf32 else ''} {ms:.2f} ms")
    del blk, z0, zw, sg, mg
    torch.cuda.empty_cache()
    return out


def config_legs(dev, with_cpu: bool, only=None):
    """The path's other specified workloads: GPU time (median of per-iteration
    events), TFLOP/s over the algorithmic flops, % of peak, the compulsory
    HBM bytes per ms of the module legs, and the CPU oracle (fp32, median of
    5 after 1 warm-up) beside them.  ``only``: the legs to run (names cfg1,
    cfg2, cfg3, fp32, fp32_tf32, cfg5), all by default."""
    if with_cpu:
        from oracle import reference as ref
    cores = cpu_threads() if with_cpu else None
    res = {}
    want = lambda name: only is None or name in only  # noqa: E731

    def cpu_leg(fn, fl):
        if not with_cpu:
            return {}
        med, ts = cpu_median(fn)
        return {"cpu_ms": round(med * 1e3, 2), "cpu_gflops": round(fl / med / 1e9, 2),
                "cpu_cores": cores, "cpu_runs_s": [round(t, 3) for t in ts]}

    if want("cfg1"):
        # cfg1: one PairformerBlock at N=128, fp32 (c_s 384, 16 single heads)
        cfg = wl.BLOCK_N128
        z, s, mask, gen = wl.make_inputs(cfg)
        blk = PairformerBlock(n_heads=16, c_z=128, c_s=384, c_hidden_mul=128,
                              c_hidden_pair_att=32, no_heads_pair=4)
        wl.init_module_(blk, gen)
        blk = blk.eval()
        p = _cpu_params(blk)
        blk = blk.to(dev)
        zg, sg, mg = z.to(dev), s.to(dev), mask.to(dev)
        f = flops(cfg.n)["block"]
        with torch.no_grad():
            ms = gpu_median_ms(lambda: blk(sg, zg, mg, triangle_multiplicative="hip",
                                           triangle_attention="hip"))
        t = f / (ms * 1e-3) / 1e12
        res["cfg1_block_n128_fp32"] = dict(
            gpu_ms=round(ms, 4), gflop=round(f / 1e9, 2), tflops=round(t, 2),
            pct_f32_peak=round(100 * t / PEAK_F32_TFLOPS, 2), dtype="fp32",
            **cpu_leg(lambda: ref.pairformer_block(s, z, mask, p), f))
        log(f"bench: cfg1 block n=128 fp32 {ms:.3f} ms")
        del blk, zg, sg, mg

    if want("cfg2"):
        # cfg2: TriangleAttention starting node at N=384, bf16 z, last 38 tokens padded
        cfg = wl.TRIATT_N384
        z, _, mask, gen = wl.make_inputs(cfg)
        mod = TriangleAttention(cfg.c_z, cfg.head_dim, cfg.heads)
        wl.init_module_(mod, gen)
        mod = mod.eval()
        p = _cpu_params(mod)
        mod = mod.to(dev)
        zb = z.to(torch.bfloat16)
        zg, mg = zb.to(dev), mask.to(dev)
        fa = flops(cfg.n)
        f = fa["core"] + fa["att_lin"]
        fn = lambda: mod(zg, mg, triangle_attention="hip")  # noqa: E731
        with torch.no_grad():
            ms = gpu_median_ms(fn)
            core_ms = kernel_avg_ms(fn, _lib.K_TRIATT_CORE)
        t, tc = f / (ms * 1e-3) / 1e12, fa["core"] / (core_ms * 1e-3) / 1e12
        zf = zb.float()
        res["cfg2_triatt_start_n384_bf16"] = dict(
            gpu_ms=round(ms, 4), gflop=round(f / 1e9, 2), tflops=round(t, 2),
            pct_bf16_peak=round(100 * t / PEAK_BF16_TFLOPS, 2),
            core_ms=round(core_ms, 4), core_tflops=round(tc, 2),
            core_pct_bf16_peak=round(100 * tc / PEAK_BF16_TFLOPS, 2),
            hbm_gbs=round((2 * cfg.n ** 2 * cfg.c_z * 2 + cfg.n ** 2 * 4) / (ms * 1e-3) / 1e9, 1),
            dtype="bf16", pad_tokens=cfg.n_pad,
            **cpu_leg(lambda: ref.triangle_attention(zf, mask, p, cfg.heads), f))
        log(f"bench: cfg2 tri-attn n=384 {ms:.3f} ms")
        del mod, zg, mg

    if want("cfg3"):
        # cfg3: TriangleMultiplication outgoing + incoming at N=768, bf16 z
        cfg = wl.TRIMUL_N768
        z, _, mask, gen = wl.make_inputs(cfg)
        mo = TriangleMultiplicationOutgoing(cfg.c_z, cfg.c_hidden_mul)
        mi = TriangleMultiplicationIncoming(cfg.c_z, cfg.c_hidden_mul)
        wl.init_module_(mo, gen)
        wl.init_module_(mi, gen)
        po, pi = _cpu_params(mo), _cpu_params(mi)
        mo, mi = mo.eval().to(dev), mi.eval().to(dev)
        zb = z.to(torch.bfloat16)
        zg, mg = zb.to(dev), mask.to(dev)
        fm = flops(cfg.n)
        f = 2 * (fm["contract"] + fm["mul_lin"])

        def fn():
            mo(zg, mg, triangle_multiplicative="hip")
            mi(zg, mg, triangle_multiplicative="hip")

        with torch.no_grad():
            ms = gpu_median_ms(fn)
            ct_ms = kernel_avg_ms(fn, _lib.K_TRIMUL_CONTRACT)
        t, tc = f / (ms * 1e-3) / 1e12, fm["contract"] / (ct_ms * 1e-3) / 1e12
        zf = zb.float()

        def cpu3():
            ref.triangle_multiplication(zf, mask, po, True)
            ref.triangle_multiplication(zf, mask, pi, False)

        res["cfg3_trimul_out_in_n768_bf16"] = dict(
            gpu_ms=round(ms, 4), gflop=round(f / 1e9, 2), tflops=round(t, 2),
            pct_bf16_peak=round(100 * t / PEAK_BF16_TFLOPS, 2),
            contract_ms=round(ct_ms, 4), contract_tflops=round(tc, 2),
            contract_pct_bf16_peak=round(100 * tc / PEAK_BF16_TFLOPS, 2),
            hbm_gbs=round(2 * (2 * cfg.n ** 2 * cfg.c_z * 2 + cfg.n ** 2 * 4) / (ms * 1e-3) / 1e9, 1),
            dtype="bf16", **cpu_leg(cpu3, f))
        log(f"bench: cfg3 tri-mul n=768 out+in {ms:.3f} ms")
        del mo, mi, zg, mg
        torch.cuda.empty_cache()

    if want("fp32"):
        res["fp32_block_n1024"] = fp32_block_leg(dev)
    if want("fp32_tf32"):
        res["fp32_tf32_block_n1024"] = fp32_block_leg(dev, tf32=True)

    if want("cfg5"):
        # cfg5: N=2048, 4 blocks with the single track (c_s 384), bench mode,
        # peak memory
        cfg = wl.STRESS_N2048
        z, s, mask, gen = wl.make_inputs(cfg)
        stack = PairformerStack(n_blocks=cfg.n_blocks, n_heads=16, c_z=cfg.c_z, c_s=cfg.c_s)
        wl.init_module_(stack, gen)
        stack = stack.eval().to(dev)
        z0, s0, mg = z.to(dev), s.to(dev), mask.to(dev)
        zw = torch.empty_like(z0)

        def stress():
            zw.copy_(z0)
            with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
                stack(s0, zw, mg, triangle_multiplicative="hip", triangle_attention="hip",
                      inplace_safe=True)

        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        ms = gpu_median_ms(stress, warm=1, iters=3)
        peak = (torch.cuda.max_memory_allocated(dev) - base) / 2 ** 30
        fb = flops(cfg.n, c_s=cfg.c_s)
        f = cfg.n_blocks * fb["block"]
        t = f / (ms * 1e-3) / 1e12
        res["cfg5_stress_4x_n2048_bf16"] = dict(
            gpu_ms=round(ms, 2), block_ms=round(ms / cfg.n_blocks, 3), gflop=round(f / 1e9, 1),
            tflops=round(t, 2), pct_bf16_peak=round(100 * t / PEAK_BF16_TFLOPS, 2),
            peak_gib_above_inputs=round(peak, 2), total_gib_in_use=round(
                torch.cuda.max_memory_allocated(dev) / 2 ** 30, 2), dtype="bf16",
            residual_dtype="fp32", c_s=cfg.c_s)
        log(f"bench: cfg5 stress n=2048 x4 {ms:.1f} ms, peak {peak:.1f} GiB")
        del stack, z0, s0, zw, mg
        torch.cuda.empty_cache()

    return res


CALIB_BYTES = 1 << 30  # bytes read (and written) by the calibration kernel


def pmc_probe(step, dev):
    """Dispatches for the HBM-traffic counters: a plain elementwise kernel
    reading CALIB_BYTES and writing CALIB_BYTES (its FETCH_SIZE / WRITE_SIZE
    give the counters' scale), then the trunk step's kernels."""
    src = torch.ones(CALIB_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    torch.add(src, 1.0, out=dst)
    torch.cuda.synchronize()
    del src, dst
    step()
    torch.cuda.synchronize()
    print("pmc probe done", flush=True)


def load_traffic(n: int):
    """HBM bytes per launch of each kernel as measured by the committed
    rocprofv3 --pmc summary for this workload (or {} if there is none)."""
    path = os.path.join(ROOT, "profiles", f"pmc_traffic_trunk_n{n}.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f).get("bytes_per_launch", {})


def layer_norm_measure(n: int, dev, reps: int = 20):
    """Standalone pair LayerNorm of the workload (N*N rows x 128, bf16, with
    weight and bias) through the fast-LayerNorm entry points: forward and
    backward average launch time from the library's HIP events, algorithmic
    HBM bytes per launch (forward: read x, write out, write mean and invvar;
    backward: read x, dout, mean and invvar, write grad_input), and torch's
    own F.layer_norm forward on the same tensor for comparison."""
    from opendde_amd import fast_layer_norm as fln
    rows, c = n * n, 128
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(rows, c, generator=g, device=dev).to(torch.bfloat16)
    dout = torch.randn(rows, c, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(c, generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn(c, generator=g, device=dev).to(torch.bfloat16)
    _, mean, invvar = fln.forward_with_both_affine(x, (c,), w, b, 1e-5)
    fln.backward_with_both_affine(dout, mean, invvar, x, (c,), w, b, 1e-5)
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    for _ in range(reps):
        fln.forward_with_both_affine(x, (c,), w, b, 1e-5)
        fln.backward_with_both_affine(dout, mean, invvar, x, (c,), w, b, 1e-5)
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    f_tot, f_cnt = _lib.timing_query(_lib.K_LAYER_NORM)
    b_tot, b_cnt = _lib.timing_query(_lib.K_LAYER_NORM_BWD)
    _lib.timing_reset()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.nn.functional.layer_norm(x, (c,), w, b, 1e-5)
    e0.record()
    for _ in range(reps):
        torch.nn.functional.layer_norm(x, (c,), w, b, 1e-5)
    e1.record()
    torch.cuda.synchronize()
    torch_ms = e0.elapsed_time(e1) / reps
    fwd_bytes = rows * c * 2 * 2 + rows * 8
    bwd_bytes = rows * c * 2 * 3 + rows * 8
    f_ms, b_ms = f_tot / f_cnt, b_tot / b_cnt
    res = {"rows": rows, "n2": c, "dtype": "bf16", "affine": "both",
           "fwd_avg_ms": round(f_ms, 4), "fwd_bytes": fwd_bytes,
           "fwd_gbs": round(fwd_bytes / (f_ms * 1e-3) / 1e9, 1),
           "bwd_avg_ms": round(b_ms, 4), "bwd_bytes": bwd_bytes,
           "bwd_gbs": round(bwd_bytes / (b_ms * 1e-3) / 1e9, 1),
           "torch_fwd_ms": round(torch_ms, 4)}
    res["fwd_pct_hbm_peak"] = round(100 * res["fwd_gbs"] / PEAK_HBM_GBS, 2)
    res["bwd_pct_hbm_peak"] = round(100 * res["bwd_gbs"] / PEAK_HBM_GBS, 2)
    del x, dout, mean, invvar
    torch.cuda.empty_cache()
    return res


def opm_measure(n: int, dev, s_rows: int = 1280, reps: int = 10):
    """The MSA module's OuterProductMean (c_m 64, c_hidden 32, c_z 128; MSA
    depth 1280, opendde/config/data.py:31) at N residues, with a random MSA
    mask and the update added into an fp32 pair tensor, bf16 arithmetic:
    average time of the library's launch scope (projection, mask norms,
    fused outer product + W_out) from its HIP events; the reference's own
    torch path on the same inputs under bf16 autocast for comparison."""
    from opendde_amd.outer_product_mean import OuterProductMean
    g = torch.Generator().manual_seed(6)
    mod = OuterProductMean(64, 128, 32)
    wl.init_module_(mod, g, 0.05)
    mod = mod.to(dev)
    m = torch.randn(s_rows, n, 64, generator=g).to(dev)
    mask = (torch.rand(s_rows, n, generator=g) > 0.1).float().to(dev)
    z = torch.randn(n, n, 128, generator=g).to(dev)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        mod.hip_apply(m, mask, out=z, add_residual=True)
        torch.cuda.synchronize()
        _lib.timing_reset()
        _lib.timing_enable(True)
        for _ in range(reps):
            mod.hip_apply(m, mask, out=z, add_residual=True)
        torch.cuda.synchronize()
        _lib.timing_enable(False)
        tot, cnt = _lib.timing_query(_lib.K_OPM)
        _lib.timing_reset()
        mod(m, mask, chunk_size=128)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(2):
            mod(m, mask, chunk_size=128)
        e1.record()
        torch.cuda.synchronize()
    torch_ms = e0.elapsed_time(e1) / 2
    ms = tot / cnt
    # projections 2*S*N*c_m*2c, outer products 2*S*N^2*c^2, W_out 2*N^2*c^2*c_z
    fl = 2.0 * s_rows * n * 64 * 64 + 2.0 * s_rows * n * n * 32 * 32 + 2.0 * n * n * 32 * 32 * 128
    res = {"n_seq": s_rows, "n_res": n, "c_m": 64, "c_hidden": 32, "c_z": 128, "dtype": "bf16",
           "avg_ms": round(ms, 4), "tflops": round(fl / ms / 1e9, 1),
           "pct_bf16_peak": round(100 * fl / ms / 1e9 / PEAK_BF16_TFLOPS, 2),
           "torch_bf16_ms": round(torch_ms, 4)}
    del m, mask, z
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--n", type=int, default=1024)
    ap.add_argument("--blocks", type=int, default=48)
    ap.add_argument("--cpu-sample-n", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-opm", action="store_true",
                    help="skip the OuterProductMean measurement")
    ap.add_argument("--no-layer-norm", action="store_true",
                    help="skip the standalone fast-LayerNorm measurement")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other specified workloads (N=128 fp32 block, N=384 "
                         "attention, N=768 multiplication, N=2048 x 4 stack)")
    ap.add_argument("--no-machine", action="store_true",
                    help="skip the MFMA-rate and HBM-copy probes")
    ap.add_argument("--preset", choices=["trunk", "opendde_v1"], default="trunk",
                    help="trunk: c_z 128, 4 triangle heads, hidden 128 (the benchmark "
                         "configuration); opendde_v1: the shipped model's pair width, c_z 384 "
                         "with hidden_scale_up (12 heads, hidden 384)")
    ap.add_argument("--leg", choices=["cfg1", "cfg2", "cfg3", "fp32", "fp32_tf32", "cfg5"],
                    help="run only this workload leg on the GPU (no CPU oracle) and print "
                         "its JSON: cfg1 N=128 block fp32, cfg2 N=384 attention, cfg3 N=768 "
                         "multiplication, fp32 the N=1024 block in fp32 arithmetic, fp32_tf32 "
                         "the same with reduced-precision products allowed, cfg5 "
                         "N=2048 x 4 blocks (for kernel traces of one leg)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: one streaming calibration kernel of known "
                         "size, then one trunk step over a single block; prints nothing else")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: this build measures the single-GPU pair-stack "
              "kernels; multi-GPU runs are not part of it.", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.leg:
        print(json.dumps(config_legs(dev, with_cpu=False, only={args.leg})), flush=True)
        return
    v1 = args.preset == "opendde_v1"
    c_z, heads, ch = (384, 12, 384) if v1 else (128, 4, 128)
    cfg = wl.PairConfig("trunk", args.n, c_z=c_z, n_blocks=args.blocks,
                        n_pad=args.n * 5 // 100, random_pad=True, seed=3)
    z0, s0, mask, gen = wl.make_inputs(cfg)
    stack = PairformerStack(n_blocks=args.blocks, c_z=c_z, c_s=384, hidden_scale_up=v1)
    wl.init_module_(stack, gen)
    stack = stack.to(dev).eval()
    z0, s0, mask = z0.to(dev), s0.to(dev), mask.to(dev)
    z = torch.empty_like(z0)

    def step():
        z.copy_(z0)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            s, _ = stack(s0, z, mask, triangle_multiplicative="hip", triangle_attention="hip",
                         inplace_safe=True)
        return s

    if args.pmc_probe:
        pmc_probe(step, dev)
        return

    log(f"bench: trunk {args.blocks} blocks n={args.n}: {args.warmup} warm-up, {args.steps} timed")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        s_out = step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    assert torch.isfinite(z).all() and torch.isfinite(s_out).all(), "non-finite trunk output"
    # per-kernel breakdown from one more step with HIP events recorded around
    # every launch on its own stream (kept out of the timed region)
    _lib.timing_reset()
    _lib.timing_enable(True)
    step()
    torch.cuda.synchronize()
    _lib.timing_enable(False)

    log(f"bench: trunk {dt * 1e3 / args.steps:.1f} ms per step")
    n = args.n
    f = flops(n, c_z=c_z, h=heads, ch=ch)
    ms_step = dt * 1e3 / args.steps
    trunk_flops = f["block"] * args.blocks
    value = trunk_flops / (ms_step * 1e-3) / 1e12

    kb = kernel_bytes(n, c_z=c_z, h=heads, ch=ch)
    kernels = {}
    for kid, name in _lib.KERNEL_NAMES.items():
        tot, cnt = _lib.timing_query(kid)
        if cnt == 0:
            continue
        avg = tot / cnt
        ent = {"launches": cnt, "avg_ms": round(avg, 4), "total_ms_per_step": round(tot, 3)}
        if name == "triatt_core":
            t = f["core"] / (avg * 1e-3) / 1e12
            ent.update(tflops=round(t, 2), pct_bf16_peak=round(100 * t / PEAK_BF16_TFLOPS, 2))
            # the rows of padded tokens keep no key: the fast core skips them
            # (their output, the mean of v, costs O(N) per row); executed work
            # counts the kept rows only
            pad = n * 5 // 100
            te = t * (n - pad) / n
            ent.update(tflops_executed=round(te, 2), rows_executed=n - pad,
                       pct_bf16_peak_executed=round(100 * te / PEAK_BF16_TFLOPS, 2))
        elif name == "trimul_contract":
            t = f["contract"] / (avg * 1e-3) / 1e12
            ent.update(tflops=round(t, 2), pct_bf16_peak=round(100 * t / PEAK_BF16_TFLOPS, 2))
        elif name == "transition":
            # the pair transition and, with a single track, the single one:
            # their flops over their launches
            per_block = cnt / args.blocks
            fl = f["trans"] + (f["single_trans"] if per_block > 1 else 0.0)
            t = fl / per_block / (avg * 1e-3) / 1e12
            ent.update(tflops=round(t, 2), pct_bf16_peak=round(100 * t / PEAK_BF16_TFLOPS, 2))
        elif name in kb:
            gbs = kb[name] / (avg * 1e-3) / 1e9
            ent.update(gbs=round(gbs, 1), pct_hbm_peak=round(100 * gbs / PEAK_HBM_GBS, 2))
        kernels[name] = ent
    # the dominant kernel among those with a rate (flops or compulsory bytes)
    rated = [k for k in kernels if "tflops" in kernels[k] or "gbs" in kernels[k]]
    dom = max(rated, key=lambda k: kernels[k]["total_ms_per_step"])
    d = kernels[dom]
    traffic = None if v1 else load_traffic(n).get(dom)
    if "tflops" in d:
        achieved = d["tflops"]
        roof = {"kernel": dom, "bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic}
    else:
        achieved = d["gbs"]
        roof = {"kernel": dom, "bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic}

    att_mod_ms = sum(kernels.get(k, {}).get("avg_ms", 0) for k in ("triatt_proj", "triatt_core", "triatt_out"))
    mul_mod_ms = sum(kernels.get(k, {}).get("avg_ms", 0) for k in ("trimul_proj", "trimul_contract", "trimul_out"))
    out = {
        "metric": "Pairformer block ms + tri-attn/tri-mul TFLOP/s (% MFMA peak) at N=1024 bf16",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"pairformer_{'opendde_v1_' if v1 else ''}trunk_"
                               f"{args.blocks}x_n{n}", "n_tokens": n,
                   "n_blocks": args.blocks, "c_z": c_z, "c_s": 384, "tri_heads": heads,
                   "head_dim": 32, "c_hidden_mul": ch, "pad_tokens": n * 5 // 100,
                   "residual_dtype": "fp32", "compute_dtype": "bf16", "seed": 3},
        "block_ms": round(ms_step / args.blocks, 3),
        "tri_attn_core_tflops": kernels.get("triatt_core", {}).get("tflops"),
        "tri_attn_core_pct_peak": kernels.get("triatt_core", {}).get("pct_bf16_peak"),
        "tri_attn_module_tflops": round((f["core"] + f["att_lin"]) / (att_mod_ms * 1e-3) / 1e12, 2)
        if att_mod_ms else None,
        "tri_mul_contract_tflops": kernels.get("trimul_contract", {}).get("tflops"),
        "tri_mul_contract_pct_peak": kernels.get("trimul_contract", {}).get("pct_bf16_peak"),
        "tri_mul_module_tflops": round((f["contract"] + f["mul_lin"]) / (mul_mod_ms * 1e-3) / 1e12, 2)
        if mul_mod_ms else None,
        "kernels": kernels,
        "roofline": roof,
        "cpu_baseline": None,
        "machine": None,
        "configs": None,
        "layer_norm": None,
        "outer_product_mean": None,
    }
    del stack, z, z0, s0
    torch.cuda.empty_cache()
    if not args.no_layer_norm:
        out["layer_norm"] = layer_norm_measure(n, dev)
        log("bench: layer norm done")
    if not args.no_opm:
        out["outer_product_mean"] = opm_measure(n, dev)
        log("bench: outer product mean done")
    if not args.no_machine:
        m = probe_machine(dev)
        out["machine"] = m
        if roof["unit"] == "TFLOP/s":
            roof["frac_of_measured_peak"] = round(roof["achieved"] / m["mfma_bf16_tflops"], 4)
            roof["measured_peak"] = m["mfma_bf16_tflops"]
        else:
            roof["frac_of_measured_peak"] = round(roof["achieved"] / m["hbm_copy_gbs"], 4)
            roof["measured_peak"] = m["hbm_copy_gbs"]
        log(f"bench: machine {m}")
    cpu = not args.no_cpu_baseline and not v1
    if not args.no_configs and not v1:
        out["configs"] = config_legs(dev, with_cpu=cpu)
    if cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_sample_n, chunk=128)
        log("bench: cpu baseline done")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
