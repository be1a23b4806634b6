#!/usr/bin/env python3
"""bench.py -- BASELINE.json's headline metric on one MI355X.

Metric: "INT8 GEMM TOPS & FP32 TFLOP/s at 1 MI355X; % of MFMA peak; GEMV HBM
GB/s". `value` is the INT8 GEMM throughput on the configuration the metric is
quoted on (gemm_bench INT8, M=N=K=2048, u8 x s8 ->
int32, per-row x per-column dequant to fp32). One step = one pass of the hot
path over the batch = one pcl_gemm_u8s8_dq call with inputs resident in HBM.
The other configurations (FP32 1024^3, 350M-class GEMMs in both dtypes and
backward layouts, grown-model prefill, decode GEMV sweeps) and the rows built
around the path (causal attention, fused epilogues, the CKP1 decode engine, the
tied head with cross-entropy) are reported under "extra", with CPU timings of
the reference (built from source) or of the oracle's restatement beside them.
"vendor_library" holds the vendor GEMM library timed on the same GEMM shapes by
a separate measurement program (drivers/gemm_yardstick.cpp), for context.
Timing loops run in C (libpcl_bench.so) between HIP events recorded on the
stream the kernels are launched on.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--primary-only] [--case NAME]
"""
import argparse
import ctypes as C
import json
import os
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "pure-c-llm_amd")
sys.path.insert(0, PKG)

METRIC = "INT8 GEMM TOPS & FP32 TFLOP/s at 1 MI355X; % of MFMA peak; GEMV HBM GB/s"
PEAK_I8_TOPS = 5033.0     # 256 CU x 2.4 GHz x 8192 OP/clk (dense)
PEAK_F32_TFLOPS = 157.3   # 256 CU x 2.4 GHz x 256 FLOP/clk (dense)
PEAK_HBM_GBS = 8000.0
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "igemm_2048_hbm_traffic.txt")


def load_bench():
    import pcl  # noqa: F401  (loads libpcl_hip.so first; raises if missing)

    path = os.path.join(PKG, "libpcl_bench.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} is not built: run `make -C pure-c-llm_amd`")
    lib = C.CDLL(path)
    d, i = C.c_double, C.c_int
    lib.pcl_bench_igemm.argtypes = [i, i, i, i, i, i, i, C.POINTER(d)]
    lib.pcl_bench_igemm_ex.argtypes = [i, i, i, i, i, i, i, C.POINTER(d), C.POINTER(d)]
    lib.pcl_bench_sgemm.argtypes = [i, i, i, i, i, i, i, i, C.POINTER(d)]
    lib.pcl_bench_gemv.argtypes = [C.POINTER(i), i, i, C.POINTER(i), C.POINTER(i), i, i, i, i, C.POINTER(d),
                                   C.POINTER(d)]
    lib.pcl_bench_gemv_group.argtypes = [C.POINTER(i), i, i, C.POINTER(i), C.POINTER(i), i, i, i, C.POINTER(d),
                                         C.POINTER(d)]
    lib.pcl_bench_attn.argtypes = [i, i, i, i, i, i, i, C.POINTER(d)]
    lib.pcl_bench_attn_bwd.argtypes = [i, i, i, i, i, i, C.POINTER(d)]
    lib.pcl_bench_attn_bwd_ex.argtypes = [i, i, i, i, i, i, i, C.POINTER(d)]
    lib.pcl_bench_sgemm_ex.argtypes = [i, i, i, i, i, i, i, i, i, C.POINTER(d)]
    lib.pcl_bench_head_ce.argtypes = [i, i, i, C.c_long, i, i, i, C.POINTER(d)]
    for f in (lib.pcl_bench_igemm, lib.pcl_bench_igemm_ex, lib.pcl_bench_sgemm, lib.pcl_bench_gemv, lib.pcl_bench_gemv_group,
              lib.pcl_bench_attn,
              lib.pcl_bench_attn_bwd, lib.pcl_bench_attn_bwd_ex, lib.pcl_bench_sgemm_ex, lib.pcl_bench_head_ce):
        f.restype = i
    return pcl, lib


def _check(pcl, st, what):
    if st != 0:
        raise RuntimeError(f"{what}: status {st}: {pcl.last_error()}")


def igemm(pcl, lib, M, N, K, out_mode, warmup, steps):
    ms = C.c_double(0)
    _check(pcl, lib.pcl_bench_igemm(M, N, K, out_mode, 1, warmup, steps, C.byref(ms)), f"igemm {M}x{N}x{K}")
    per = ms.value / steps
    return {"M": M, "N": N, "K": K, "ms": round(per, 5),
            "TOPS": round(2.0 * M * N * K / (per * 1e-3) / 1e12, 1),
            "frac_peak": round(2.0 * M * N * K / (per * 1e-3) / 1e12 / PEAK_I8_TOPS, 4)}


def sgemm(pcl, lib, opA, opB, M, N, K, accumulate, warmup, steps):
    ms = C.c_double(0)
    _check(pcl, lib.pcl_bench_sgemm(opA, opB, M, N, K, accumulate, warmup, steps, C.byref(ms)),
           f"sgemm {M}x{N}x{K}")
    per = ms.value / steps
    tf = 2.0 * M * N * K / (per * 1e-3) / 1e12
    return {"M": M, "N": N, "K": K, "layout": "NT"[opA] + "NT"[opB], "ms": round(per, 5),
            "TFLOPS": round(tf, 2), "frac_peak": round(tf / PEAK_F32_TFLOPS, 4)}


def gemv(pcl, lib, kind, M, shapes, copies, warmup, steps, graph=False):
    """One sweep = one call per (K, N) shape; kind 0/1/2 = FP32 W (K x N),
    FP32 W (N x K), INT8 packed (a list gives one kind per shape). graph=True
    captures each weight copy's sweep once and replays it (one launch)."""
    kinds = kind if isinstance(kind, (list, tuple)) else [kind] * len(shapes)
    Kd = (C.c_int * len(shapes))(*kinds)
    Ks = (C.c_int * len(shapes))(*[k for k, _ in shapes])
    Ns = (C.c_int * len(shapes))(*[n for _, n in shapes])
    ms, by = C.c_double(0), C.c_double(0)
    _check(pcl, lib.pcl_bench_gemv(Kd, M, len(shapes), Ks, Ns, copies, warmup, steps, int(graph), C.byref(ms),
                                   C.byref(by)), f"gemv kinds {sorted(set(kinds))}")
    per = ms.value / steps
    gbs = by.value / (per * 1e-3) / 1e9
    return {"M": M, "ms_per_sweep": round(per, 5), "bytes_per_sweep": int(by.value), "GBps": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "weight_copies": copies, "graph": bool(graph)}


def gemv_group(pcl, lib, kind, M, shapes, copies, warmup, steps):
    """The same sweep as gemv(), every product independent, as one grouped
    launch per step (pcl_gemv_group_run)."""
    kinds = kind if isinstance(kind, (list, tuple)) else [kind] * len(shapes)
    Kd = (C.c_int * len(shapes))(*kinds)
    Ks = (C.c_int * len(shapes))(*[k for k, _ in shapes])
    Ns = (C.c_int * len(shapes))(*[n for _, n in shapes])
    ms, by = C.c_double(0), C.c_double(0)
    _check(pcl, lib.pcl_bench_gemv_group(Kd, M, len(shapes), Ks, Ns, copies, warmup, steps, C.byref(ms),
                                         C.byref(by)), f"gemv group kinds {sorted(set(kinds))}")
    per = ms.value / steps
    gbs = by.value / (per * 1e-3) / 1e9
    return {"M": M, "ms_per_sweep": round(per, 5), "bytes_per_sweep": int(by.value), "GBps": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "weight_copies": copies, "launches_per_sweep": 1}


def attn(pcl, lib, B, T, H, dh, with_probs, warmup, steps):
    """Causal attention forward. Algorithmic FLOPs: QK^T and PV over the causal
    triangle including the diagonal, 4*B*H*dh*T(T+1)/2. With probabilities the
    two-pass kernel issues 1.5x that on the matrix cores (the scores are
    computed in both passes); without, the one-pass kernel issues 1.0x."""
    ms = C.c_double(0)
    _check(pcl, lib.pcl_bench_attn(B, T, H, dh, int(with_probs), warmup, steps, C.byref(ms)),
           f"attn B{B} T{T} H{H} dh{dh}")
    per = ms.value / steps
    flops = 4.0 * B * H * dh * T * (T + 1) / 2
    tf = flops / (per * 1e-3) / 1e12
    probs_bytes = 4.0 * B * H * T * T if with_probs else 0.0
    return {"B": B, "T": T, "H": H, "dh": dh, "probs": bool(with_probs), "ms": round(per, 5),
            "TFLOPS": round(tf, 2), "frac_peak": round(tf / PEAK_F32_TFLOPS, 4),
            "mfma_TFLOPS_issued": round((1.5 if with_probs else 1.0) * tf, 2),
            "probs_GBps": round(probs_bytes / (per * 1e-3) / 1e9, 1)}


def attn_bwd(pcl, lib, B, T, H, dh, warmup, steps, with_att=False):
    """Causal attention backward from stored probabilities. Algorithmic FLOPs:
    dV, dP, dQ, dK over the causal triangle, 8*B*H*dh*T(T+1)/2. From P alone
    dP is issued twice (1.25x) and P read three times; handed the forward's
    output (pcl_attn_bwd_ex) dP is issued once (1.0x) and P read twice; dS is
    written once and read once."""
    ms = C.c_double(0)
    _check(pcl, lib.pcl_bench_attn_bwd_ex(B, T, H, dh, int(with_att), warmup, steps, C.byref(ms)),
           f"attn_bwd B{B} T{T} H{H} dh{dh}")
    per = ms.value / steps
    flops = 8.0 * B * H * dh * T * (T + 1) / 2
    tf = flops / (per * 1e-3) / 1e12
    tt_bytes = (4 if with_att else 5) * 4.0 * B * H * T * (T + 1) / 2
    return {"B": B, "T": T, "H": H, "dh": dh, "with_att": bool(with_att), "ms": round(per, 5),
            "TFLOPS": round(tf, 2), "frac_peak": round(tf / PEAK_F32_TFLOPS, 4),
            "mfma_TFLOPS_issued": round((1.0 if with_att else 1.25) * tf, 2),
            "causal_TT_GBps": round(tt_bytes / (per * 1e-3) / 1e9, 1)}


def sgemm_epi(pcl, lib, opA, opB, M, N, K, epi, warmup, steps):
    """Product + epilogue, fused (one kernel) against the reference's two-pass
    sequence (GEMM, then the elementwise kernel)."""
    out = {"M": M, "N": N, "K": K, "layout": "NT"[opA] + "NT"[opB],
           "epilogue": {1: "gelu", 2: "residual", 3: "gelu_bwd"}[epi]}
    for fused in (1, 0):
        ms = C.c_double(0)
        _check(pcl, lib.pcl_bench_sgemm_ex(opA, opB, M, N, K, epi, fused, warmup, steps, C.byref(ms)),
               f"sgemm_ex {M}x{N}x{K} epi {epi}")
        per = ms.value / steps
        out["fused_ms" if fused else "two_pass_ms"] = round(per, 5)
        out["fused_TFLOPS" if fused else "two_pass_TFLOPS"] = round(2.0 * M * N * K / (per * 1e-3) / 1e12, 2)
    out["speedup"] = round(out["two_pass_ms"] / out["fused_ms"], 3)
    return out


def head_ce(pcl, lib, M, D, V, chunk_bytes, warmup, steps):
    """The tied head fused with cross-entropy (pcl_head_ce: logits, softmax
    cross-entropy in place, d_lnf, dwte) against its cross-entropy pass alone.
    FLOPs: three M x D x V products, 6*M*D*V; the cross-entropy pass moves
    3 * 4 * M * V bytes (two reads of the logits, one write)."""
    out = {"M": M, "D": D, "V": V, "chunk_MB": round(chunk_bytes / 2 ** 20) if chunk_bytes > 0 else "1024 (default)"}
    ms = C.c_double(0)
    _check(pcl, lib.pcl_bench_head_ce(M, D, V, chunk_bytes, 0, warmup, steps, C.byref(ms)), f"head_ce {M}x{D}x{V}")
    per = ms.value / steps
    out["ms"] = round(per, 4)
    out["TFLOPS"] = round(6.0 * M * D * V / (per * 1e-3) / 1e12, 2)
    out["frac_peak"] = round(out["TFLOPS"] / PEAK_F32_TFLOPS, 4)
    ms = C.c_double(0)
    _check(pcl, lib.pcl_bench_head_ce(M, D, V, 0, 1, warmup, steps, C.byref(ms)), f"cross_entropy {M}x{V}")
    per = ms.value / steps
    out["ce_ms"] = round(per, 4)
    out["ce_GBps"] = round(12.0 * M * V / (per * 1e-3) / 1e9, 1)
    out["ce_share"] = round(out["ce_ms"] / out["ms"], 4)
    return out


def _write_ckp1(path, blk, d, h, df, nl, v, seed, wstd=0.02):
    """A CKP1 checkpoint (train.c:633-648: int[8] header, then the tensors in
    registration order) of synthetic weights: gains 1 + N(0, 0.1), biases
    N(0, 0.02), matrices N(0, wstd), embeddings N(0, 0.1)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    kinds = [("e", v * d), ("e", blk * d)]
    for _ in range(nl):
        kinds += [("g", d), ("b", d)] + [("w", d * d), ("b", d)] * 4 + \
                 [("g", d), ("b", d), ("w", d * df), ("b", df), ("w", df * d), ("b", d)]
    kinds += [("g", d), ("b", d)]
    with open(path, "wb") as f:
        f.write(np.array([0x434B5031, blk, d, h, df, nl, v, 0], "<i4").tobytes())
        for kind, n in kinds:
            mean, std = {"g": (1.0, 0.1), "b": (0.0, 0.02), "w": (0.0, wstd), "e": (0.0, 0.1)}[kind]
            f.write(rng.normal(mean, std, n).astype("<f4").tobytes())


def decode_e2e(pcl, dims=(256, 512, 16, 2048, 16, 2048), n_new=255, ref_tokens=24, modes=(0, 1)):
    """Greedy decoding of a synthetic CKP1 checkpoint of the grown model
    (block 256, d 512, 16 heads, d_ff 2048, 16 layers, vocab 2048): one prompt
    token then n_new tokens fed back on the GPU, eagerly and as one graph
    replay per token, with fp32 weights and with INT8 weights
    (pcl_model_load_ex); beside it the reference generate.c forward (built from
    source in oracle/_ref, OpenMP on all host cores) on the same checkpoint."""
    import tempfile

    import numpy as np

    blk, d, h, df, nl, v = dims
    tmp = tempfile.mkdtemp(prefix="pcl_ckp1_")
    path = os.path.join(tmp, "grown.ckp1")
    _write_ckp1(path, blk, d, h, df, nl, v, seed=77, wstd=0.05)
    out = {"model": f"block {blk}, d_model {d}, heads {h}, d_ff {df}, layers {nl}, vocab {v}",
           "weights_MB": round(4.0 * (v * d + blk * d + nl * (4 * d * d + 2 * d * df)) / 1e6, 1)}
    for weights, wtag in ((pcl.W_FP32, ""), (pcl.W_INT8, "int8_")):
        m = pcl.lib.pcl_model_load_ex(path.encode(), weights)
        if not m:
            raise RuntimeError(f"pcl_model_load_ex: {pcl.last_error()}")
        try:
            prompt = np.array([1], np.int32)
            toks = np.empty(n_new, np.int32)
            for graph in modes:
                _check(pcl, pcl.lib.pcl_model_generate(m, pcl.ptr(prompt), 1, n_new, pcl.ptr(toks), graph),
                       "generate")
                t0 = time.perf_counter()
                _check(pcl, pcl.lib.pcl_model_generate(m, pcl.ptr(prompt), 1, n_new, pcl.ptr(toks), graph),
                       "generate")
                dt = time.perf_counter() - t0
                tag = wtag + ("graph" if graph else "eager")
                out[f"{tag}_tokens_per_s"] = round(n_new / dt, 1)
                out[f"{tag}_ms_per_token"] = round(1e3 * dt / n_new, 4)
        finally:
            pcl.lib.pcl_model_free(m)
    gen = None
    if ref_tokens > 0:  # the CPU reference leg
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import binding as ob
        gen = ob.ref("libref_generate.so")
    if gen is not None:
        gen.pcl_ref_gen_load(path.encode())
        logits = np.empty(v, np.float32)
        tok = 1
        t0 = time.perf_counter()
        for pos in range(ref_tokens):
            gen.pcl_ref_gen_forward(tok, pos, ob.p(logits))
            tok = int(np.argmax(logits))
        dt = time.perf_counter() - t0
        out["cpu_reference_tokens_per_s"] = round(ref_tokens / dt, 1)
        out["cpu_reference_sample"] = (f"generate.c forward, positions 0..{ref_tokens - 1}, "
                                       f"OpenMP threads {os.environ.get('OMP_NUM_THREADS', 'default')}")
    try:
        os.remove(path)
        os.rmdir(tmp)
    except OSError:
        pass
    return out


def read_trace_us():
    """Average duration of the headline kernel in the committed rocprofv3
    kernel trace of this same bench command (profiles/), in microseconds."""
    path = os.path.join(ROOT, "profiles", "igemm_2048_kernel_trace.txt")
    if not os.path.exists(path):
        return None
    m = re.search(r"^\s*average\s*:\s*([0-9.]+) ns", open(path).read(), re.M)
    return round(float(m.group(1)) / 1e3, 3) if m else None


def read_traffic():
    """HBM bytes per launch of the primary kernel, measured by rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, calibrated on a copy of known size) and recorded
    in profiles/; None when no such measurement has been committed."""
    if not os.path.exists(PROFILE_TRAFFIC):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(PROFILE_TRAFFIC).read(), re.M)
    return float(m.group(1)) if m else None


def host_cores():
    """Threads this process may use on the host: the affinity mask, capped by
    OMP_NUM_THREADS where the GPU boxes set it (the box's share of the host)."""
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return min(cores, share) if share > 0 else cores


def _vnni_operands(ob, np, M, N, K, seed):
    """u8 activations, s8 weights in gemm_bench's VNNI panel layout
    (gemm_bench.c:254), corr = 128*colsum and dq, as gemm_bench prepares them
    offline (untimed, gemm_bench.c:368, 379-381)."""
    Au = ob.u8((M, K), seed)
    Bq = ob.s8((K, N), seed + 1)
    Bp = np.empty((N // 16) * (K // 4) * 64, np.int8)
    for j in range(4):
        Bp.reshape(N // 16, K // 4, 16, 4)[:, :, :, j] = Bq[j::4, :].reshape(K // 4, N // 16, 16).transpose(1, 0, 2)
    corr = (128 * Bq.astype(np.int64).sum(0)).astype(np.int32)
    dq = ob.uniform((N,), seed + 3, 1e-3, 1e-2)
    return Au, Bp, corr, dq


def host_share(threads):
    """What the host lends this process: the cgroup CPU quota (cpu.max), the
    load average, and the share of `threads` hardware threads the timed CPU
    runs actually obtained (process CPU time over wall time x threads). A box
    whose host is busy with other tenants shows a low share; it is why the
    same CPU rung reads differently from box to box."""
    out = {"threads": threads}
    try:
        q, per = open("/sys/fs/cgroup/cpu.max").read().split()
        out["cgroup_cpu_max"] = "unlimited" if q == "max" else round(int(q) / int(per), 2)
    except (OSError, ValueError):
        out["cgroup_cpu_max"] = "unreadable"
    try:
        out["loadavg_1m"] = round(os.getloadavg()[0], 2)
    except OSError:
        pass
    out["online_cpus"] = os.cpu_count()
    return out


def cpu_reference(M=2048, N=2048, K=2048):
    """The reference's CPU path timed on this host (oracle/_ref builds of
    gemm_bench.c and tensor.c from source; kind "reference"), best of 6 runs
    as gemm_bench.c:329-337 (packing and quantisation untimed, :368, 379-381):
      * the VNNI INT8 rung (gemm_int8_kernel, gemm_bench.c:260-285) on the
        primary 2048^3 problem, single-threaded as in gemm_bench and driven over
        M bands by 4, 8 and all host threads (1 and 4 threads on a 512-row
        sample, scaled per operation);
      * the same rung on the 350M-class shapes, full 4096 rows at all threads,
        and on the tied head 4096 x 50257 x 1024 (a 512-row sample; N padded to
        50272, the 16-column VNNI panel of gemm_bench.c:254);
      * FP32 v3-MT (gemm_packed_mt, :167-192) on both gemm_bench configs
        (1024^3 and M 1024, K 1024, N 4096, gemm_bench.c:413-414) at 1, 4, 8
        and all threads, and on the 350M-class forward shapes (full 4096 rows)
        at all threads;
      * v1 i-k-j as tensor.c's OpenMP matmul (tensor.c:34-53) on 1024^3;
      * the reference's own 1-core roofs (:287-325);
      * the host share the runs obtained (host_share).
    Returns (cpu_baseline, detail); cpu_baseline is None when the reference
    build is unusable on this host."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import binding as ob

    gb = ob.ref("libref_gemm_bench.so")
    if gb is None or not gb.pcl_ref_cpu_ok():
        return None, {"unavailable": "reference build missing or the host lacks AVX-512 VNNI (gemm_bench.c:25)"}
    cores = host_cores()
    thr = sorted({1, 4, 8, cores})
    detail = {"cpu": cpu_model(), "cores": cores}
    share = host_share(cores)
    cpu_s, wall_s = [0.0], [0.0]

    def best(f, reps=6, threads=1):
        t = 1e30
        for _ in range(reps):
            c0, t0 = time.process_time(), time.perf_counter()
            f()
            dt = time.perf_counter() - t0
            if threads == cores:
                cpu_s[0] += time.process_time() - c0
                wall_s[0] += dt * cores
            t = min(t, dt)
        return t

    Au, Bp, corr, dq = _vnni_operands(ob, np, M, N, K, 11)
    Cm = np.empty((M, N), np.float32)
    i8 = {}
    for t in thr:
        rows = M if t >= 8 else 512
        dt = best(lambda: gb.pcl_ref_gemm_int8_mt(t, ob.p(Au), K, ob.p(Bp), ob.p(corr), ob.p(dq), ob.p(Cm), rows, N),
                  threads=t)
        i8[f"{t}t"] = round(2.0 * rows * N * K / dt / 1e12, 4)
    detail["int8_vnni_2048_TOPS"] = i8
    shapes = {"qkv": (4096, 1024, 3072), "attn_out": (4096, 1024, 1024), "ffn_up": (4096, 1024, 4096),
              "ffn_down": (4096, 4096, 1024), "head": (512, 1024, 50272)}
    i8s = {}
    for name, (m, k, n) in shapes.items():
        A2, B2, c2, d2 = _vnni_operands(ob, np, m, n, k, 21)
        C2 = np.empty((m, n), np.float32)
        dt = best(lambda: gb.pcl_ref_gemm_int8_mt(cores, ob.p(A2), k, ob.p(B2), ob.p(c2), ob.p(d2), ob.p(C2), m, n),
                  threads=cores)
        i8s[name] = round(2.0 * m * n * k / dt / 1e12, 4)
        del A2, B2, C2
    detail[f"int8_vnni_350m_TOPS_{cores}t"] = i8s
    mm = ob.ref("libref_model.so")
    v1 = {}
    for (m, k, n) in ((1024, 1024, 1024), (1024, 1024, 4096)):
        A, B = ob.frand((m, k), 1234), ob.frand((k, n), 1235)
        Cf = np.empty((m, n), np.float32)
        v3 = {}
        for t in thr:
            gb.pcl_ref_set_threads(t)
            v3[f"{t}t"] = round(2.0 * m * n * k / best(lambda: gb.pcl_ref_gemm_packed_mt(ob.p(A), ob.p(B), ob.p(Cf),
                                                                                         m, k, n), threads=t) / 1e9, 1)
            if mm is not None and n == 1024:
                v1[f"{t}t"] = round(2.0 * m * n * k / best(lambda: mm.matmul(ob.p(A), ob.p(B), ob.p(Cf), m, k, n),
                                                           3, threads=t) / 1e9, 1)
        detail[f"fp32_v3mt_{m}x{k}x{n}_GFLOPS"] = v3
    detail["fp32_v1_ikj_tensor_matmul_1024_GFLOPS"] = v1
    gb.pcl_ref_set_threads(cores)
    f3 = {}
    for name, (m, k, n) in shapes.items():
        if name == "head":
            continue
        A, B = ob.frand((m, k), 1236), ob.frand((k, n), 1237)
        Cf = np.empty((m, n), np.float32)
        f3[name] = round(2.0 * m * n * k / best(lambda: gb.pcl_ref_gemm_packed_mt(ob.p(A), ob.p(B), ob.p(Cf), m, k, n),
                                                threads=cores) / 1e9, 1)
    detail[f"fp32_v3mt_350m_GFLOPS_{cores}t"] = f3
    gb.pcl_ref_set_threads(1)
    detail["roofs_1core"] = {"fp32_GFLOPS": round(gb.pcl_ref_peak_gflops(), 1),
                             "int8_GOPS": round(gb.pcl_ref_peak_int8_gops(), 1)}
    share["obtained"] = round(cpu_s[0] / wall_s[0], 3) if wall_s[0] > 0 else None
    detail["host_share"] = share
    base = {"value": i8[f"{cores}t"], "unit": "TOP/s", "cores": cores, "kind": "reference",
            "sample": f"full {M}x{N}x{K} u8 x s8 problem through the reference gemm_int8_kernel (AVX-512 VNNI, "
                      f"gemm_bench.c:260-285) over M bands on {cores} host threads, best of 6; the runs at "
                      f"{cores} threads obtained {share['obtained']} of them (process CPU time / wall x threads)"}
    return base, detail


# Single configurations for profiling runs (bench.py --case NAME): the same
# timing loops as the full run, one configuration per process.
DECODE_LAYER = [(512, 1536), (512, 512), (512, 2048), (2048, 512)]
INT8_350M = {"qkv": (4096, 3072, 1024), "attn_out": (4096, 1024, 1024), "ffn_up": (4096, 4096, 1024),
             "ffn_down": (4096, 1024, 4096), "head": (4096, 50257, 1024)}
CASES = {
    "int8_2048": lambda pcl, lib, w, s: igemm(pcl, lib, 2048, 2048, 2048, 2, w, s),
    "int8_qkv": lambda pcl, lib, w, s: igemm(pcl, lib, 4096, 3072, 1024, 2, w, s),
    "int8_ffn_up": lambda pcl, lib, w, s: igemm(pcl, lib, 4096, 4096, 1024, 2, w, s),
    "int8_ffn_down": lambda pcl, lib, w, s: igemm(pcl, lib, 4096, 1024, 4096, 2, w, s),
    "int8_head": lambda pcl, lib, w, s: igemm(pcl, lib, 4096, 50257, 1024, 2, w, s),
    "fp32_1024": lambda pcl, lib, w, s: sgemm(pcl, lib, 0, 0, 1024, 1024, 1024, 0, w, s),
    "fp32_ffn_up": lambda pcl, lib, w, s: sgemm(pcl, lib, 0, 0, 4096, 4096, 1024, 0, w, s),
    "fp32_qkv": lambda pcl, lib, w, s: sgemm(pcl, lib, 0, 0, 4096, 3072, 1024, 0, w, s),
    "fp32_qkv_nt": lambda pcl, lib, w, s: sgemm(pcl, lib, 0, 1, 4096, 3072, 1024, 0, w, s),
    "fp32_attn_out": lambda pcl, lib, w, s: sgemm(pcl, lib, 0, 0, 4096, 1024, 1024, 0, w, s),
    "fp32_ffn_down": lambda pcl, lib, w, s: sgemm(pcl, lib, 0, 0, 4096, 1024, 4096, 0, w, s),
    "fp32_bwd_dx_nt": lambda pcl, lib, w, s: sgemm(pcl, lib, 0, 1, 4096, 1024, 4096, 1, w, s),
    "fp32_bwd_dw_tn": lambda pcl, lib, w, s: sgemm(pcl, lib, 1, 0, 1024, 4096, 4096, 1, w, s),
    "epi_350m_ffn_down_resid": lambda pcl, lib, w, s: sgemm_epi(pcl, lib, 0, 0, 4096, 1024, 4096, 2, w, s),
    "epi_350m_ffn_up_gelu": lambda pcl, lib, w, s: sgemm_epi(pcl, lib, 0, 0, 4096, 4096, 1024, 1, w, s),
    "decode_e2e": lambda pcl, lib, w, s: decode_e2e(pcl),
    # eager steps only (kernel traces: rocprofv3 does not follow graph launches here)
    "decode_e2e_eager": lambda pcl, lib, w, s: decode_e2e(pcl, ref_tokens=0, modes=(0,)),
    "head_ce_350m": lambda pcl, lib, w, s: head_ce(pcl, lib, 4096, 1024, 50257, 0, w, s),
    "head_ce_350m_chunk128": lambda pcl, lib, w, s: head_ce(pcl, lib, 4096, 1024, 50257, 128 << 20, w, s),
    "attn_350m": lambda pcl, lib, w, s: attn(pcl, lib, 4, 1024, 16, 64, True, w, s),
    "attn_350m_noprobs": lambda pcl, lib, w, s: attn(pcl, lib, 4, 1024, 16, 64, False, w, s),
    "attn_trainer_dh128": lambda pcl, lib, w, s: attn(pcl, lib, 4, 1024, 12, 128, True, w, s),
    "attn_bwd_350m": lambda pcl, lib, w, s: attn_bwd(pcl, lib, 4, 1024, 16, 64, w, s),
    "attn_bwd_350m_with_att": lambda pcl, lib, w, s: attn_bwd(pcl, lib, 4, 1024, 16, 64, w, s, True),
    "attn_bwd_trainer_dh128": lambda pcl, lib, w, s: attn_bwd(pcl, lib, 4, 1024, 12, 128, w, s),
    "gemv_head_fp32_m1": lambda pcl, lib, w, s: gemv(pcl, lib, 1, 1, [(1024, 50257)], 3, w, s),
    "gemv_head_int8_m1": lambda pcl, lib, w, s: gemv(pcl, lib, 2, 1, [(1024, 50257)], 11, w, s),
    "gemv_head_fp32_m8": lambda pcl, lib, w, s: gemv(pcl, lib, 1, 8, [(1024, 50257)], 3, w, s),
    "gemv_head_int8_m8": lambda pcl, lib, w, s: gemv(pcl, lib, 2, 8, [(1024, 50257)], 11, w, s),
    "gemv_head_int8_m2": lambda pcl, lib, w, s: gemv(pcl, lib, 2, 2, [(1024, 50257)], 11, w, s),
    "gemv_head_int8_m3": lambda pcl, lib, w, s: gemv(pcl, lib, 2, 3, [(1024, 50257)], 11, w, s),
    "gemv_head_int8_m4": lambda pcl, lib, w, s: gemv(pcl, lib, 2, 4, [(1024, 50257)], 11, w, s),
    "decode_int8_m1": lambda pcl, lib, w, s: gemv(pcl, lib, 2, 1, DECODE_LAYER * 16 + [(512, 2048)], 11, w, s),
    "decode_int8_m4": lambda pcl, lib, w, s: gemv(pcl, lib, 2, 4, DECODE_LAYER * 16 + [(512, 2048)], 11, w, s),
    "decode_fp32_m1": lambda pcl, lib, w, s: gemv(pcl, lib, [0] * 64 + [1], 1, DECODE_LAYER * 16 + [(512, 2048)],
                                                   3, w, s),
    "decode_group_fp32_m1": lambda pcl, lib, w, s: gemv_group(pcl, lib, [0] * 64 + [1], 1,
                                                               DECODE_LAYER * 16 + [(512, 2048)], 3, w, s),
    "decode_group_fp32_m4": lambda pcl, lib, w, s: gemv_group(pcl, lib, [0] * 64 + [1], 4,
                                                               DECODE_LAYER * 16 + [(512, 2048)], 3, w, s),
    "decode_group_fp32_m8": lambda pcl, lib, w, s: gemv_group(pcl, lib, [0] * 64 + [1], 8,
                                                               DECODE_LAYER * 16 + [(512, 2048)], 3, w, s),
    "decode_group_int8_m1": lambda pcl, lib, w, s: gemv_group(pcl, lib, 2, 1, DECODE_LAYER * 16 + [(512, 2048)],
                                                               11, w, s),
    "decode_group_int8_m4": lambda pcl, lib, w, s: gemv_group(pcl, lib, 2, 4, DECODE_LAYER * 16 + [(512, 2048)],
                                                               11, w, s),
    # one weight copy (52 / 206 MB): the sweep reads the Infinity Cache, not HBM
    "decode_group_int8_m1_1copy": lambda pcl, lib, w, s: gemv_group(pcl, lib, 2, 1,
                                                                     DECODE_LAYER * 16 + [(512, 2048)], 1, w, s),
    "decode_group_fp32_m1_1copy": lambda pcl, lib, w, s: gemv_group(pcl, lib, [0] * 64 + [1], 1,
                                                                     DECODE_LAYER * 16 + [(512, 2048)], 1, w, s),
    "decode_group_int8_m8": lambda pcl, lib, w, s: gemv_group(pcl, lib, 2, 8, DECODE_LAYER * 16 + [(512, 2048)],
                                                               11, w, s),
    "gemv_group_head_int8_m1": lambda pcl, lib, w, s: gemv_group(pcl, lib, 2, 1, [(1024, 50257)], 11, w, s),
    "gemv_group_head_int8_m8": lambda pcl, lib, w, s: gemv_group(pcl, lib, 2, 8, [(1024, 50257)], 11, w, s),
    "gemv_group_head_fp32_m1": lambda pcl, lib, w, s: gemv_group(pcl, lib, 1, 1, [(1024, 50257)], 3, w, s),
}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_next_rows():
    """The oracle's restatements of the reference functions behind the "next"
    rows, timed on the host beside their GPU numbers (kind "port": train.c is
    built here only at small compile-time dims): the tied head + cross-entropy
    forward and backward (train.c:412-465, OpenMP over rows / vocabulary as in
    train.c) on 4 token rows of the 350M shape, and causal attention forward
    and backward (train.c:339-407, one thread) on one sequence-head of it."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import binding as ob

    out = {"kind": "port", "omp_threads": os.environ.get("OMP_NUM_THREADS", "default")}
    M, D, V = 4, 1024, 50257
    x = ob.normal((M, D), 501, 0.0, 1.0)
    w = ob.normal((V, D), 502, 0.0, 0.05)
    t = (np.arange(M) * 7919 % V).astype(np.int32)
    t0 = time.perf_counter()
    ob.head_ce(x, w, t)
    dt = time.perf_counter() - t0
    out["head_ce_350m"] = {"sample": f"{M} of the 4096 token rows (D 1024, V 50257), forward + backward",
                           "ms_per_row": round(1e3 * dt / M, 2),
                           "ms_4096_rows_scaled": round(1e3 * dt / M * 4096, 1)}
    T, dh = 1024, 64
    q, k, v = (ob.normal((T, dh), 510 + i, 0.0, 1.0) for i in range(3))
    t0 = time.perf_counter()
    att, probs = ob.attention_forward(q, k, v, 1, T, 1, dh)
    t1 = time.perf_counter()
    ob.attention_backward(ob.normal((T, dh), 513, 0.0, 1.0), q, k, v, probs, 1, T, 1, dh)
    t2 = time.perf_counter()
    out["attn_350m"] = {"sample": "1 of the 64 sequence-heads (T 1024, d_head 64)",
                        "fwd_ms_per_head": round(1e3 * (t1 - t0), 2),
                        "bwd_ms_per_head": round(1e3 * (t2 - t1), 2),
                        "fwd_ms_64_heads_scaled": round(1e3 * (t1 - t0) * 64, 1),
                        "bwd_ms_64_heads_scaled": round(1e3 * (t2 - t1) * 64, 1)}
    return out


# Compulsory bytes of the INT8 350M-class products (M x K u8 +
# K x N s8 + 4 M N fp32 out + scales), for the attainable roof min(peak, I x HBM)
def _i8_attainable(M, N, K):
    ops = 2.0 * M * N * K
    byts = M * K + K * N + 4.0 * M * N + 4.0 * (M + N)
    return min(PEAK_I8_TOPS, ops / byts * PEAK_HBM_GBS / 1e3)


def measured_roofs(pcl):
    """The part's own roofs (pcl_measure_peak_mfma / pcl_measure_bandwidth,
    gemm_bench.c:195-210 and 287-325 on the GPU)."""
    d = C.c_double
    out = {}
    for key, data in (("mfma_i8_random_TOPS", 0), ("mfma_i8_zero_TOPS", 1), ("mfma_f32_random_TFLOPS", 2)):
        r = d(0)
        pcl.check(pcl.lib.pcl_measure_peak_mfma(data, C.byref(r)))
        out[key] = round(r.value, 1)
    g = (d * 4)()
    pcl.check(pcl.lib.pcl_measure_bandwidth(512 << 20, g))
    for n, key in enumerate(("hbm_triad_GBps", "hbm_copy_GBps", "hbm_read_GBps", "hbm_write_GBps")):
        out[key] = round(g[n], 1)
    # the INT8 kernels' operand feed (L2 -> LDS) on the one-tile-per-CU grids,
    # and the floor it sets on their K loop at the feed's own clock
    for key, (m, n, k) in (("2048", (2048, 2048, 2048)), ("ffn_down", (4096, 1024, 4096))):
        r = d(0)
        pcl.check(pcl.lib.pcl_measure_lds_feed(m, n, k, C.byref(r)))
        out[f"int8_tile_feed_{key}_GBps"] = round(r.value, 1)
        out[f"int8_tile_feed_{key}_loop_floor_us"] = round((m // 128) * (n // 128) * 256.0 * k / (r.value * 1e3), 2)
        # the same stream read into registers: is the ceiling the DMA or L2 -> CU?
        pcl.check(pcl.lib.pcl_measure_tile_read(m, n, k, C.byref(r)))
        out[f"int8_tile_read_vgpr_{key}_GBps"] = round(r.value, 1)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--primary-only", action="store_true", help="time only the headline kernel (profiling runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run device-to-device copies of this size (HBM counter calibration)")
    ap.add_argument("--case", choices=sorted(CASES),
                    help="time only this configuration and print its numbers (profiling runs)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (it runs the per-GPU shard "
              "of the path on one GPU). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    pcl, lib = load_bench()
    pcl.check(pcl.lib.pcl_init())
    info = pcl.device_info()
    if args.case:
        res = CASES[args.case](pcl, lib, args.warmup, args.steps)
        if args.calib_copy_mib:
            nb = args.calib_copy_mib << 20
            src, dst = pcl.DeviceBuffer(nb), pcl.DeviceBuffer(nb)
            for _ in range(3):
                pcl.check(pcl.lib.pcl_memcpy_d2d(dst.ptr, src.ptr, nb))
            res["calib_copy_bytes"] = nb
        print(json.dumps({"case": args.case, "steps": args.steps, "warmup": args.warmup, **res}), flush=True)
        return
    M = N = K = 2048
    ops = 2.0 * M * N * K
    pcl.sync()
    t0 = time.perf_counter()
    ms, us_each = C.c_double(0), C.c_double(0)
    _check(pcl, lib.pcl_bench_igemm_ex(M, N, K, 2, 1, args.warmup, args.steps, C.byref(ms), C.byref(us_each)),
           "igemm 2048^3")
    wall = time.perf_counter() - t0
    per = ms.value / args.steps
    tops = round(ops / (per * 1e-3) / 1e12, 1)
    roofs = measured_roofs(pcl)
    out = {
        "metric": METRIC,
        "value": tops,
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (xorshift32 u8 activations, s8 weights, scales U[1e-3,1e-2])",
        "config": {"workload": "gemm_bench INT8 GEMM M=N=K=2048, u8 x s8 -> int32, per-row x per-column dequant "
                               "to fp32 (BASELINE.json configs[1])",
                   "M": M, "N": N, "K": K,
                   "kernel": "igemm_kg_kernel<4,2,1> (one 128x128 tile per workgroup, 2 producer waves filling "
                             "a 4-deep LDS ring by DMA, 8 consumer waves on v_mfma_i32_16x16x64_i8)",
                   "parallelism": "single GPU",
                   "warmup_min_ms": 20},
        "roofline": {"bound": "mfma", "achieved": tops, "peak": PEAK_I8_TOPS, "unit": "TOP/s",
                     "frac": round(tops / PEAK_I8_TOPS, 4), "traffic": read_traffic(),
                     "trace_kernel_us": read_trace_us(),
                     "isolated_launch_us": round(us_each.value, 3),
                     "frac_of_measured_i8_mfma": round(tops / roofs["mfma_i8_random_TOPS"], 4),
                     "algorithmic_ops_per_launch": int(ops),
                     "algorithmic_bytes_per_launch": M * K + K * N + 4 * M * N + 4 * (M + N)},
        "measured_roofs": roofs,
        "device": info,
        "timed_wall_s": round(wall, 3),
    }
    if args.calib_copy_mib:
        nb = args.calib_copy_mib << 20
        src, dst = pcl.DeviceBuffer(nb), pcl.DeviceBuffer(nb)
        for _ in range(3):
            pcl.check(pcl.lib.pcl_memcpy_d2d(dst.ptr, src.ptr, nb))
        out["calib_copy_bytes"] = nb
    ex = {}
    if not args.primary_only:
        ex = run_rows(pcl, lib)
        out["rows"] = compact_rows(ex, roofs)
        ys = vendor_yardstick()
        if ys is not None:
            out["vendor_library"] = ys
    if not args.no_cpu_baseline:
        base, cpu = cpu_reference(M, N, K)
        if base is not None:
            out["cpu_baseline"] = base
        if not args.primary_only:
            ex["cpu_reference"] = cpu
            ex["cpu_port_next_rows"] = cpu_next_rows()
            out["cpu"] = {k: v for k, v in cpu.items() if k != "roofs_1core"}
    if ex:
        # the full tables: one JSON line on stderr (stdout carries the one result line)
        print("bench_detail " + json.dumps(ex), file=sys.stderr, flush=True)
    print(json.dumps(out), flush=True)


def vendor_yardstick():
    """The vendor GEMM library (hipBLASLt) timed beside libpcl_hip on the
    gemm_bench and 350M-class shapes, by a separate measurement program
    (drivers/gemm_yardstick.cpp, run after this process's own timed work):
    context for the fractions of the datasheet peak. libpcl_hip never links
    the vendor library. None when the program is not built."""
    exe = os.path.join(PKG, "build", "gemm_yardstick")
    if not os.path.exists(exe):
        return None
    try:
        r = subprocess.run([exe], capture_output=True, text=True, timeout=240)
    except (OSError, subprocess.TimeoutExpired):
        return None
    for line in r.stdout.splitlines():
        if line.startswith("yardstick_json "):
            return json.loads(line[len("yardstick_json "):])
    return None


def run_rows(pcl, lib):
    """Every configuration beside the headline, at the bench's own step counts."""
    w, s = 5, 20

    class Rows(dict):  # a progress line on stderr as each row finishes
        def __setitem__(self, k, v):
            super().__setitem__(k, v)
            print(f"bench: {k} done", file=sys.stderr, flush=True)

    ex = Rows()
    ex["fp32_gemm_1024"] = sgemm(pcl, lib, 0, 0, 1024, 1024, 1024, 0, w, 50)
    ex["int8_350m"] = {name: igemm(pcl, lib, m, n, k, 2, w, s) for name, (m, n, k) in INT8_350M.items()}
    ex["fp32_350m"] = {name: sgemm(pcl, lib, a, b, m, n, k, acc, w, s) for name, (a, b, m, n, k, acc) in {
        "qkv": (0, 0, 4096, 3072, 1024, 0), "attn_out": (0, 0, 4096, 1024, 1024, 0),
        "ffn_up": (0, 0, 4096, 4096, 1024, 0), "ffn_down": (0, 0, 4096, 1024, 4096, 0),
        "head_nt": (0, 1, 4096, 50257, 1024, 0),
        "bwd_dX_ffn_up_nt": (0, 1, 4096, 1024, 4096, 1), "bwd_dW_ffn_up_tn": (1, 0, 1024, 4096, 4096, 1)}.items()}
    ex["grown_prefill_t256"] = {
        "fp32": {name: sgemm(pcl, lib, a, b, m, n, k, 0, w, 50) for name, (a, b, m, n, k) in {
            "qkv": (0, 0, 256, 1536, 512), "attn_out": (0, 0, 256, 512, 512), "ffn_up": (0, 0, 256, 2048, 512),
            "ffn_down": (0, 0, 256, 512, 2048), "head_nt": (0, 1, 256, 2048, 512)}.items()},
        "int8": {name: igemm(pcl, lib, m, n, k, 2, w, 50) for name, (m, n, k) in {
            "qkv": (256, 1536, 512), "attn_out": (256, 512, 512), "ffn_up": (256, 2048, 512),
            "ffn_down": (256, 512, 2048), "head": (256, 2048, 512)}.items()},
    }
    # One decode sweep of the grown model: 16 layers (K x N weights) + the tied
    # head (N x K). FP32 205 MB per sweep, 3 rotating weight copies (> the
    # 256 MB Infinity Cache); INT8 51 MB, 11 copies. Per product: one call per
    # product (the dependent decode chain's launch pattern), eager and as one
    # captured graph; grouped: the 65 independent products in one launch.
    fp32_step = DECODE_LAYER * 16 + [(512, 2048)]
    fp32_kinds = [0] * (len(DECODE_LAYER) * 16) + [1]
    dec = {}
    for Mt in (1, 4, 8):
        dec[f"fp32_M{Mt}"] = gemv(pcl, lib, fp32_kinds, Mt, fp32_step, 3, 2, 10)
        dec[f"fp32_M{Mt}_graph"] = gemv(pcl, lib, fp32_kinds, Mt, fp32_step, 3, 2, 10, graph=True)
        dec[f"fp32_M{Mt}_grouped"] = gemv_group(pcl, lib, fp32_kinds, Mt, fp32_step, 3, 3, 30)
        dec[f"int8_M{Mt}"] = gemv(pcl, lib, 2, Mt, fp32_step, 11, 2, 10)
        dec[f"int8_M{Mt}_graph"] = gemv(pcl, lib, 2, Mt, fp32_step, 11, 2, 10, graph=True)
        dec[f"int8_M{Mt}_grouped"] = gemv_group(pcl, lib, 2, Mt, fp32_step, 11, 3, 30)
    ex["grown_decode_gemv"] = dec
    ex["decode_e2e_grown"] = decode_e2e(pcl)
    ex["head_350m_gemv_fp32"] = {f"M{Mt}": gemv(pcl, lib, 1, Mt, [(1024, 50257)], 3, 2, 20) for Mt in (1, 8)}
    ex["head_350m_gemv_int8"] = {f"M{Mt}": gemv(pcl, lib, 2, Mt, [(1024, 50257)], 11, 2, 20) for Mt in (1, 8)}
    ex["fp32_350m_epilogues"] = {
        "ffn_up_gelu": sgemm_epi(pcl, lib, 0, 0, 4096, 4096, 1024, 1, w, s),
        "attn_out_residual": sgemm_epi(pcl, lib, 0, 0, 4096, 1024, 1024, 2, w, s),
        "ffn_down_residual": sgemm_epi(pcl, lib, 0, 0, 4096, 1024, 4096, 2, w, s),
        "bwd_dX_ffn_down_gelu_bwd": sgemm_epi(pcl, lib, 0, 1, 4096, 4096, 1024, 3, w, s),
    }
    ex["head_ce"] = {
        "350m": head_ce(pcl, lib, 4096, 1024, 50257, 0, 1, max(2, s // 20)),
        "350m_chunk_128MB": head_ce(pcl, lib, 4096, 1024, 50257, 128 << 20, 1, max(2, s // 20)),
        "grown_t256": head_ce(pcl, lib, 256, 512, 2048, 0, 3, 50),
    }
    ex["attn_fwd"] = {
        "350m_probs": attn(pcl, lib, 4, 1024, 16, 64, True, w, s),
        "350m_no_probs": attn(pcl, lib, 4, 1024, 16, 64, False, w, s),
        "trainer_dh128_probs": attn(pcl, lib, 4, 1024, 12, 128, True, w, s),
        "grown_t256_probs": attn(pcl, lib, 1, 256, 16, 32, True, w, 50),
    }
    ex["attn_bwd"] = {
        "350m": attn_bwd(pcl, lib, 4, 1024, 16, 64, w, s),
        "350m_with_att": attn_bwd(pcl, lib, 4, 1024, 16, 64, w, s, True),
        "trainer_dh128": attn_bwd(pcl, lib, 4, 1024, 12, 128, w, s),
        "grown_t256": attn_bwd(pcl, lib, 1, 256, 16, 32, w, 50),
    }
    return dict(ex)


def compact_rows(ex, roofs):
    """The north-star rows and the next rows in a few hundred bytes each:
    [rate, fraction of the datasheet peak, fraction of the attainable roof]."""
    r = {}
    r["int8_350m_TOPS"] = {"cols": ["TOPS", "frac_peak", "frac_attainable", "frac_measured_mfma"]}
    for name, (m, n, k) in INT8_350M.items():
        t = ex["int8_350m"][name]["TOPS"]
        r["int8_350m_TOPS"][name] = [t, round(t / PEAK_I8_TOPS, 3), round(t / _i8_attainable(m, n, k), 3),
                                     round(t / roofs["mfma_i8_random_TOPS"], 3)]
    r["fp32_350m_TFLOPS"] = {"cols": ["TFLOPS", "frac_peak", "frac_measured_mfma"]}
    for name, v in ex["fp32_350m"].items():
        r["fp32_350m_TFLOPS"][name] = [v["TFLOPS"], v["frac_peak"], round(v["TFLOPS"] / roofs["mfma_f32_random_TFLOPS"], 3)]
    v = ex["fp32_gemm_1024"]
    r["fp32_1024_TFLOPS"] = [v["TFLOPS"], v["frac_peak"]]
    r["grown_prefill_us"] = {dt: {k: round(1e3 * q["ms"], 2) for k, q in ex["grown_prefill_t256"][dt].items()}
                             for dt in ("fp32", "int8")}
    d = ex["grown_decode_gemv"]
    r["grown_decode_sweep_GBps"] = {"cols": ["per_product", "per_product_graph", "grouped", "grouped_frac_hbm"]}
    for key in ("fp32_M1", "fp32_M4", "fp32_M8", "int8_M1", "int8_M4", "int8_M8"):
        g = d[key + "_grouped"]
        r["grown_decode_sweep_GBps"][key] = [d[key]["GBps"], d[key + "_graph"]["GBps"], g["GBps"], g["frac_hbm"]]
    r["head_350m_gemv_GBps"] = {f"{dt}_{m}": [ex[f"head_350m_gemv_{dt}"][m]["GBps"], ex[f"head_350m_gemv_{dt}"][m]["frac_hbm"]]
                                for dt in ("fp32", "int8") for m in ("M1", "M8")}
    r["attn_350m_TFLOPS"] = {"fwd_probs": ex["attn_fwd"]["350m_probs"]["TFLOPS"],
                             "fwd_one_pass": ex["attn_fwd"]["350m_no_probs"]["TFLOPS"],
                             "bwd": ex["attn_bwd"]["350m"]["TFLOPS"],
                             "bwd_with_att": ex["attn_bwd"]["350m_with_att"]["TFLOPS"]}
    r["head_ce_350m"] = {"TFLOPS": ex["head_ce"]["350m"]["TFLOPS"], "ms": ex["head_ce"]["350m"]["ms"]}
    e = ex["decode_e2e_grown"]
    r["decode_e2e_grown_tok_s"] = {"fp32": e.get("eager_tokens_per_s"), "fp32_graph": e.get("graph_tokens_per_s"),
                                   "int8": e.get("int8_eager_tokens_per_s"),
                                   "int8_graph": e.get("int8_graph_tokens_per_s"),
                                   "cpu_reference": e.get("cpu_reference_tokens_per_s")}
    r["epilogue_speedup"] = {k: v["speedup"] for k, v in ex["fp32_350m_epilogues"].items()}
    return r


if __name__ == "__main__":
    main()
