"""Benchmark of the W4A8 linear path (rotation + per-token int8 quant + int4 x int8 GEMM).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload of ``value`` (one "step"): one Qwen3-8B decoder layer's seven
quantized linears (q/o 4096->4096, k/v 4096->1024, gate/up 4096->12288,
down 12288->4096) at M = 1 decode token, bf16 in and out.  As in a decoder
layer, q/k/v read one input (the attention input) and gate/up another (the
MLP input); each trio / pair runs as one group (paroquant::w4a8_linear_group:
one rotation launch + one GEMM launch), o and down alone (two launches each).
The same layer with all seven linears called separately is reported next to
it.  A pool of distinct layers (8 by
default, 772 MB of weights, so the 256 MB Infinity Cache cannot serve them)
is captured as ONE HIP graph, the way a model's decode step is captured
whole; a replay is as many steps as the pool has layers, and exactly
--steps steps are timed (whole replays plus a graph of the remaining
layers) after exactly --warmup untimed ones.  value = algorithmic bytes
of the layer / time per step, in GB/s, where per linear
  B = N*K/2 + 2*N*K/128 + N*K/256 + 3*8*K + 2*K + 2*M*K + 2*M*N.
Also reported: M = 4 and 16 decode, M = 3072 prefill in int8 TOPS and % of
the 5.0 POPS dense int8 peak, a speculative-decoding verify block (36 chained
layers at M = 16 with bf16 RMSNorm between the attention and MLP linears), a
ragged packed batch (8 requests of U{1..512} tokens), the roofline of the
dominant kernel (the decode GEMM at M = 1) and the CPU oracle timed on the
host.

Every timed region except the headline decode one follows at least
--warm-seconds of untimed replays (the shader clock settles under sustained
load); the headline keeps exactly --warmup untimed steps.

Data are synthetic (seeded), weights random-init; one process, one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
COPY_CAL_BYTES = 256 << 20
# HBM bytes per launch of a kernel, measured with rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes and calibrated on a copy of known size; each summary (with
# the commands that made it) holds the figure on a "traffic_bytes_per_launch:" line.
TRAFFIC_SUMMARIES = {
    "decode_gemm_M1_layer": os.path.join(ROOT, "profiles", "decode_m1_layer_gemm_hbm_traffic.md"),
    "decode_split_rotation_M1_layer": os.path.join(ROOT, "profiles", "decode_m1_layer_gemm_hbm_traffic.md"),
    "decode_gemm_int8_a_M1": os.path.join(ROOT, "profiles", "decode_gemm_m1_hbm_traffic.md"),
    "prefill_gemm_M3072": os.path.join(ROOT, "profiles", "prefill_m3072_gemm_hbm_traffic.md"),
}


def measured_traffic(name):
    """The summary's traffic_bytes_per_launch figure for kernel `name` (a line "traffic_bytes_per_launch:"
    or "traffic_bytes_per_launch[name]:"), or None."""
    try:
        for line in open(TRAFFIC_SUMMARIES[name]):
            if line.startswith(f"traffic_bytes_per_launch[{name}]:") or (
                    line.startswith("traffic_bytes_per_launch:") and name == "decode_gemm_int8_a_M1"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None
INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0
KROT = 8


def linear_bytes(M: int, N: int, K: int) -> int:
    return N * K // 2 + 2 * N * K // 128 + N * K // 256 + 3 * KROT * K + 2 * K + 2 * M * K + 2 * M * N


def gemm_kernel_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic bytes of the GEMM kernel alone: int4 codes, fp16 scales, int4 zeros,
    int8 activations + fp32 token scales in, bf16 out."""
    return N * K // 2 + 2 * N * K // 128 + N * K // 256 + M * K + 4 * M + 2 * M * N


def rotated_gemm_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic bytes of the decode GEMM that quantizes its A operand itself: int4 codes, fp16 scales,
    int4 zeros, the rotated fp16 rows and their fp32 group maxima in, bf16 out."""
    return N * K // 2 + 2 * N * K // 128 + N * K // 256 + 2 * M * K + 4 * M * K // 128 + 2 * M * N


def split_rotation_bytes(M: int, K: int, members: int) -> int:
    """Algorithmic bytes of one split-rotation launch for `members` linears over one bf16 input: x read once;
    per member its rotation parameters (fp16 angles, int16 pairs, fp16 channel scales) in, its rotated fp16
    rows and fp32 group maxima out."""
    return 2 * M * K + members * (3 * KROT * K + 2 * K + 2 * M * K + 4 * M * K // 128)


def w16_linear_bytes(M: int, N: int, K: int) -> int:
    """W4A16 linear: int4 codes, fp16 scale + scaled zero per (group, column), rotation operands, fp16 in/out."""
    return N * K // 2 + 4 * N * K // 128 + 3 * KROT * K + 2 * K + 2 * M * K + 2 * M * N


def w16_gemm_bytes(M: int, N: int, K: int) -> int:
    """W4A16 GEMM kernel alone: int4 codes, fp16 s and sz, fp16 activations in, fp16 out."""
    return N * K // 2 + 4 * N * K // 128 + 2 * M * K + 2 * M * N


def w16_meta(wmeta):
    """s | sz << 16 metadata of the W4A16 GEMM for the weights behind a W4A8 wmeta (s | z << 16), with
    sz = fp16(-(s * z)) as WQLinear stores it; the packed codes are shared."""
    import torch

    s_bits = (wmeta & 0xFFFF).long()
    z = ((wmeta >> 16) & 0xF).float()
    s = torch.where(s_bits >= 32768, s_bits - 65536, s_bits).to(torch.int16).view(torch.float16).float()
    sz_bits = (-(s * z)).to(torch.float16).view(torch.int16).long() & 0xFFFF
    m = s_bits | (sz_bits << 16)
    return torch.where(m >= 2 ** 31, m - 2 ** 32, m).to(torch.int32).contiguous()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pool-layers", type=int, default=8)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-verify", action="store_true", help="skip the 36-layer speculative verify block (M = 16)")
    ap.add_argument("--no-ragged", action="store_true", help="skip the ragged packed batch")
    ap.add_argument("--no-w4a16", action="store_true", help="skip the W4A16 (WQLinear) figures")
    ap.add_argument("--no-mxfp4", action="store_true", help="skip the fused rotation + MXFP4 figures")
    ap.add_argument("--no-separate", action="store_true",
                    help="skip the decode layers with all seven linears called separately (so that a kernel "
                         "trace's rotation and quantizing-GEMM launches all come from the grouped layer and its "
                         "two-stage graphs)")
    ap.add_argument("--no-decode-per-shape", action="store_true",
                    help="skip the per-shape decode GEMM timing (so that a kernel trace's int8-A decode GEMM "
                         "launches all come from the roofline graph)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--warm-seconds", type=float, default=0.3,
                    help="minimum wall time of untimed replays before each timed region")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first copy 256 MiB device to device 3 times: the known-size kernel that calibrates "
                         "the FETCH_SIZE / WRITE_SIZE counter passes")
    ap.add_argument("--library-gemms", action="store_true",
                    help="measurement mode: also time the vendor library's plain GEMMs at the M = 3072 shapes "
                         "(torch._int_mm int8 -> int32, torch._scaled_mm fp8 -> bf16, bf16 matmul; hipBLASLt) "
                         "beside this build's W4A8 GEMM")
    ap.add_argument("--decode-m", type=str, default="1,4,16",
                    help="comma-separated decode token counts to time (M = 1 gives value)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        return 2

    import torch

    import alpamayo_amd  # noqa: F401
    from alpamayo_amd import _lib, workloads

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.ones(COPY_CAL_BYTES // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    names = list(workloads.QWEN3_8B_LINEARS)
    shapes = [workloads.QWEN3_8B_LINEARS[n] for n in names]

    # ---- weight pool -------------------------------------------------------
    t0 = time.time()
    pool = []
    for li in range(args.pool_layers):
        g = workloads.generator(1001 + li, device=dev)
        layer = [workloads.build_module(workloads.linear_spec(n, N, K, g, device=dev), dev)
                 for n, (N, K) in zip(names, shapes)]
        pool.append(layer)
    torch.cuda.synchronize()
    from alpamayo_amd.quantization import SharedInputRotateLinears
    # q/k/v read the attention input and gate/up the MLP input: each trio / pair runs as one group
    groups = [(SharedInputRotateLinears(L[0:3]), SharedInputRotateLinears(L[4:6])) for L in pool]
    pool_mb = sum(m.rotate_linear.qlinear.qweight.numel() for L in pool for m in L) / 1e6
    log(f"pool: {args.pool_layers} layers, {pool_mb:.0f} MB of packed int4 weights ({time.time() - t0:.1f}s)")

    def make_inputs(M, seed):
        """Per layer: the attention input (q, k, v), the attention output (o), the MLP input (gate, up) and
        the activated MLP hidden state (down)."""
        g = workloads.generator(seed, device=dev)
        return [tuple(workloads.activations(M, K, g, device=dev) for K in (4096, 4096, 4096, 12288)) for _ in pool]

    def run_layer(li, X, grouped):
        L = pool[li]
        xa, xo, xm, xd = X
        if grouped:
            qkv, gu = groups[li]
            return [*qkv(xa), L[3](xo), *gu(xm), L[6](xd)]
        return [L[0](xa), L[1](xa), L[2](xa), L[3](xo), L[4](xm), L[5](xm), L[6](xd)]

    def capture_layers(M, seed, grouped, n_layers=None):
        """One HIP graph holding the pool's layers (the first n_layers of them) in sequence, as a
        model's decode step is captured whole: a replay is that many steps."""
        xs = make_inputs(M, seed)[:n_layers]
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for li, X in enumerate(xs):
                run_layer(li, X, grouped)
        torch.cuda.current_stream().wait_stream(s)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            outs = [run_layer(li, X, grouped) for li, X in enumerate(xs)]
        return gr, outs, xs

    def time_exact_steps(M, seed, grouped, steps, warmup):
        """Exactly `warmup` untimed then exactly `steps` timed layer steps: whole replays of the pool graph plus
        one replay of a graph of the first (steps mod pool) layers.  Returns ms per step."""
        P = len(pool)
        full, _, _ = capture_layers(M, seed, grouped)
        parts = {}
        for r in {steps % P, warmup % P} - {0}:
            parts[r], _, _ = capture_layers(M, seed, grouped, r)

        def run(n):
            for _ in range(n // P):
                full.replay()
            if n % P:
                parts[n % P].replay()

        run(warmup)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run(steps)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def time_graphs(graphs, steps, warmup, warm_s=None):
        # warm up for at least warm_s (default --warm-seconds) of wall time as well as `warmup`
        # replays: the GPU's clock takes a few hundred ms of sustained load to settle, and a
        # short compute-bound run timed before that reads several percent slow
        warm_s = args.warm_seconds if warm_s is None else warm_s
        t0, i = time.perf_counter(), 0
        while i < warmup or time.perf_counter() - t0 < warm_s:
            graphs[i % len(graphs)].replay()
            i += 1
            if i % len(graphs) == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            graphs[i % len(graphs)].replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps          # ms per step

    result = {}

    # ---- decode: M = 1 (value), 4, 16 -------------------------------------
    # Each M twice: q/k/v and gate/up as groups over their shared inputs (value), and all seven
    # linears as separate calls.
    decode, decode_sep = {}, {}
    decode_ms = sorted({int(v) for v in args.decode_m.split(",")} | {1})
    P = len(pool)
    for M in decode_ms:
        b = sum(linear_bytes(M, N, K) for N, K in shapes)
        for grouped, table in ((True, decode), (False, decode_sep)):
            if not grouped and args.no_separate:
                continue
            ms = time_exact_steps(M, 5000 + M, grouped, args.steps, args.warmup)
            table[M] = (ms, b / (ms * 1e-3) / 1e9)
            log(f"decode M={M} {'grouped ' if grouped else 'separate'}: {ms * 1e3:.1f} us/layer, "
                f"{table[M][1]:.0f} GB/s")
    ms_per_step, value = decode[1]

    # ---- the headline layer's own kernels, each timed alone ----------------
    # The grouped M = 1 layer in its two stages (pq_w4a8_linear_group_stage): all rotation launches
    # (rotate_split_kernel) of the pool captured as one graph, all GEMM launches (gemm_skinny quantizing its
    # A operand itself, from the rotated row the first stage left in the workspace) as another,
    # each launch with exactly the configuration the layer runs.  Per launch: the GEMM moves its members'
    # packed weights, scales and zeros, their rotated fp16 rows and group maxima, and writes bf16 y; the
    # rotation reads x once and each member's parameters and writes its rotated fp16 rows and group maxima.
    Mh = 1
    stage_calls = []
    for li, (xa, xo, xm, xd) in enumerate(make_inputs(Mh, 7002)):
        L = pool[li]
        for mods, x in ((L[0:3], xa), (L[3:4], xo), (L[4:6], xm), (L[6:7], xd)):
            rls = [m.rotate_linear for m in mods]
            st = alpamayo_amd.ops.W4A8GroupStages(
                x, [r.rotation.rot_idx for r in rls], [r.rotation.rot_cs for r in rls],
                [r.rotation.scales_f32 for r in rls], rls[0].rotation.krot, [r.qlinear.qweight for r in rls],
                [r.qlinear.scales for r in rls], [r.qlinear.bias for r in rls], True, True, torch.bfloat16)
            stage_calls.append((st, [(r.qlinear.out_features, r.qlinear.in_features) for r in rls]))

    def capture_calls(fn):
        s2 = torch.cuda.Stream()
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s2):
            fn()
        torch.cuda.current_stream().wait_stream(s2)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return g

    g_rot = capture_calls(lambda: [st.rotate() for st, _ in stage_calls])
    g_gemm = capture_calls(lambda: [st.gemm() for st, _ in stage_calls])
    n_calls = len(stage_calls)
    hrot_ms = time_graphs([g_rot], max(10, args.steps // 10), 3)
    hgemm_ms = time_graphs([g_gemm], max(10, args.steps // 10), 3)
    del g_rot, g_gemm
    hgemm_bytes = sum(rotated_gemm_bytes(Mh, N, K) for _, shp in stage_calls for N, K in shp)
    hrot_bytes = sum(split_rotation_bytes(Mh, shp[0][1], len(shp)) for _, shp in stage_calls)
    hgemm_us = hgemm_ms * 1e3 / n_calls
    hrot_us = hrot_ms * 1e3 / n_calls
    hgemm_gbs = hgemm_bytes / (hgemm_ms * 1e-3) / 1e9
    hrot_gbs = hrot_bytes / (hrot_ms * 1e-3) / 1e9
    log(f"headline layer M=1, GEMM launches alone: {hgemm_us:.2f} us/launch avg, {hgemm_gbs:.0f} GB/s; "
        f"rotation launches alone: {hrot_us:.2f} us/launch avg, {hrot_gbs:.0f} GB/s")
    del stage_calls

    # ---- the decode GEMM on int8 activations at M = 1 ---------------------
    xq_all = []
    for L, (xa, xo, xm, xd) in zip(pool, make_inputs(1, 7001)):
        row = []
        for m, x in zip(L, (xa, xa, xa, xo, xm, xm, xd)):
            r = m.rotate_linear.rotation
            row.append(torch.ops.paroquant.rotate_quant_i8(x, r.rot_idx, r.rot_cs, r.scales_f32, r.krot, True, True))
        xq_all.append(row)
    gemm_launches = [(m.rotate_linear.qlinear, xq, xs) for L, row in zip(pool, xq_all) for m, (xq, xs) in zip(L, row)]
    gg = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for q, xq, xs in gemm_launches:
            torch.ops.paroquant.w4a8_gemm(xq, xs, q.qweight, q.scales, None, torch.bfloat16)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(gg):
        for q, xq, xs in gemm_launches:
            torch.ops.paroquant.w4a8_gemm(xq, xs, q.qweight, q.scales, None, torch.bfloat16)
    gemm_ms = time_graphs([gg], max(10, args.steps // 10), 3)
    gemm_bytes = sum(gemm_kernel_bytes(1, q.out_features, q.in_features) for q, _, _ in gemm_launches)
    achieved = gemm_bytes / (gemm_ms * 1e-3) / 1e9
    per_launch_us = gemm_ms * 1e3 / len(gemm_launches)
    log(f"decode GEMM M=1: {per_launch_us:.2f} us/launch avg, {achieved:.0f} GB/s")
    del gg
    # the same launches one shape at a time (q/o, k/v, gate/up: 16 per replay; down: 8)
    gemm_per_shape = None if args.no_decode_per_shape else {}
    for shape in ([] if args.no_decode_per_shape else sorted({(q.out_features, q.in_features)
                                                              for q, _, _ in gemm_launches})):
        sel = [t for t in gemm_launches if (t[0].out_features, t[0].in_features) == shape]
        g1 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g1):
            for q, xq, xs in sel:
                torch.ops.paroquant.w4a8_gemm(xq, xs, q.qweight, q.scales, None, torch.bfloat16)
        sus = time_graphs([g1], max(10, args.steps // 10), 3) * 1e3 / len(sel)
        sb = gemm_kernel_bytes(1, *shape)
        gemm_per_shape[f"{shape[0]}x{shape[1]}"] = {"us_per_launch": round(sus, 2),
                                                   "GBps": round(sb / (sus * 1e-6) / 1e9, 1),
                                                   "frac_hbm": round(sb / (sus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del g1
    if gemm_per_shape is not None:
        log("decode GEMM M=1 per shape (N x K): " + ", ".join(f"{k} {v['us_per_launch']} us ({v['GBps']:.0f} GB/s)"
                                                              for k, v in gemm_per_shape.items()))

    # ---- prefill M = 3072 ---------------------------------------------------
    prefill = None
    if not args.no_prefill:
        M = 3072
        g = workloads.generator(6000, device=dev)
        X = tuple(workloads.activations(M, K, g, device=dev) for K in (4096, 4096, 4096, 12288))
        ops = sum(2 * M * N * K for N, K in shapes)
        res = {}
        for grouped in (True, False):
            run_layer(0, X, grouped)
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                outs = run_layer(0, X, grouped)
            res[grouped] = time_graphs([gr], args.prefill_steps, 3)
            del gr, outs
        ms = res[True]
        tops = ops / (ms * 1e-3) / 1e12
        tops_sep = ops / (res[False] * 1e-3) / 1e12
        # GEMM kernels alone (each linear's GEMM on its own)
        L = pool[0]
        xq = []
        for m, x in zip(L, (X[0], X[0], X[0], X[1], X[2], X[2], X[3])):
            r = m.rotate_linear.rotation
            xq.append(torch.ops.paroquant.rotate_quant_i8(x, r.rot_idx, r.rot_cs, r.scales_f32, r.krot, True, True))
        gg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gg):
            for m, (q8, s8) in zip(L, xq):
                q = m.rotate_linear.qlinear
                torch.ops.paroquant.w4a8_gemm(q8, s8, q.qweight, q.scales, None, torch.bfloat16)
        gms = time_graphs([gg], args.prefill_steps, 3)
        gtops = ops / (gms * 1e-3) / 1e12
        # each shape's GEMM alone (q, k, gate, down; o, v, up repeat a shape): REP launches per graph,
        # so that the gap between two graph replays is not charged to one kernel
        REP = 4
        per_shape = {}
        for idx in (0, 1, 4, 6):
            m = L[idx]
            q = m.rotate_linear.qlinear
            q8, s8 = xq[idx]
            g1 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g1):
                for _ in range(REP):
                    torch.ops.paroquant.w4a8_gemm(q8, s8, q.qweight, q.scales, None, torch.bfloat16)
            sms = time_graphs([g1], args.prefill_steps, 3) / REP
            sops = 2 * M * q.out_features * q.in_features
            per_shape[f"{q.out_features}x{q.in_features}"] = {
                "us": round(sms * 1e3, 1), "pct_int8_peak": round(100 * sops / (sms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 2)}
            del g1
        log("prefill GEMM per shape (N x K): " + ", ".join(f"{k} {v['us']} us ({v['pct_int8_peak']}%)"
                                                           for k, v in per_shape.items()))
        # the rotate + int8 quant launch of one linear alone (bf16 rows in, int8 codes + token scales out)
        rq_shape = {}
        for idx in (0, 6):
            r = L[idx].rotate_linear.rotation
            x = (X[0], X[0], X[0], X[1], X[2], X[2], X[3])[idx]
            K = x.shape[-1]
            g1 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g1):
                for _ in range(REP):
                    torch.ops.paroquant.rotate_quant_i8(x, r.rot_idx, r.rot_cs, r.scales_f32, r.krot, True, True)
            sms = time_graphs([g1], args.prefill_steps, 3) / REP
            gbps = (2 * M * K + M * K + 4 * M) / (sms * 1e-3) / 1e9
            rq_shape[str(K)] = {"us": round(sms * 1e3, 1), "GBps": round(gbps, 1),
                                "frac_hbm": round(gbps / HBM_PEAK_GBS, 4)}
            del g1
        log("prefill rotate+quant per K: " + ", ".join(f"K={k} {v['us']} us ({v['GBps']} GB/s)"
                                                       for k, v in rq_shape.items()))
        prefill_ops = ops
        prefill = {"ms_per_layer": round(ms, 4), "tops": round(tops, 1), "gemm_only_ms": round(gms, 5),
                   "pct_int8_peak": round(100 * tops / INT8_PEAK_TOPS, 2),
                   "separate_linears_ms_per_layer": round(res[False], 4), "separate_linears_tops": round(tops_sep, 1),
                   "gemm_only_tops": round(gtops, 1), "gemm_only_pct_int8_peak": round(100 * gtops / INT8_PEAK_TOPS, 2),
                   "gemm_per_shape": per_shape, "rotate_quant_per_K": rq_shape}
        log(f"prefill M=3072: {ms:.3f} ms/layer grouped, {tops:.0f} TOPS ({prefill['pct_int8_peak']}%); "
            f"separate {res[False]:.3f} ms/layer, {tops_sep:.0f} TOPS; GEMMs alone {gtops:.0f} TOPS")
        del gg, xq, X

    # ---- the vendor library's plain GEMMs at the prefill shapes (measurement mode) ----
    # What a dense GEMM without int4 unpacking or group scales sustains on this GPU: int8 x int8 -> int32
    # (torch._int_mm), fp8 e4m3 x fp8 -> bf16 (torch._scaled_mm, unit scales) and bf16 (torch.matmul), B
    # column-major (the weight [N, K] transposed); four launches per captured graph.
    libg = None
    if args.library_gemms:
        libg = {}
        M = 3072
        for N, K in sorted(set(shapes)):
            a8 = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev)
            w8 = torch.randint(-8, 8, (N, K), dtype=torch.int8, device=dev)
            af = torch.randn(M, K, device=dev).to(torch.float8_e4m3fn)
            wf = torch.randn(N, K, device=dev).to(torch.float8_e4m3fn)
            ab = torch.randn(M, K, device=dev, dtype=torch.bfloat16)
            wb = torch.randn(N, K, device=dev, dtype=torch.bfloat16)
            one = torch.ones((), device=dev)
            row = {}
            for name, fn, peak in (("int8_int_mm", lambda: torch._int_mm(a8, w8.t()), INT8_PEAK_TOPS),
                                   ("fp8_scaled_mm", lambda: torch._scaled_mm(af, wf.t(), scale_a=one, scale_b=one,
                                                                              out_dtype=torch.bfloat16),
                                    INT8_PEAK_TOPS),
                                   ("bf16_matmul", lambda: torch.matmul(ab, wb.t()), FP16_PEAK_TFLOPS)):
                fn()
                g1 = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g1):
                    for _ in range(4):
                        fn()
                us = time_graphs([g1], args.prefill_steps, 3) / 4 * 1e3
                row[name] = {"us": round(us, 1), "pct_peak": round(100 * 2 * M * N * K / (us * 1e-6) / 1e12 / peak, 2)}
                del g1
            libg[f"{N}x{K}"] = row
            log(f"library GEMMs M={M} N={N} K={K}: " + ", ".join(f"{k} {v['us']} us ({v['pct_peak']}%)"
                                                                for k, v in row.items()))
            del a8, w8, af, wf, ab, wb

    # ---- speculative verify block: 36 chained layers at M = 16 -------------
    # Per layer a -> (q, k, v) = L(a); o = L_o(q); h = RMSNorm_bf16(a + o) (eps 1e-6, weight U(0.8, 1.2));
    # d = L_down(silu(L_gate(h)) * L_up(h)); next a = h + d.  The norm and its residual add run inside the
    # gate/up group's rotation launch, silu * mul inside the down linear's, the h + d add inside the next
    # layer's q/k/v rotation.  Fresh random int4 weights per layer; the whole block is captured as one
    # graph.  Reported: time per verified block, and the 252 quantized linears of the
    # block alone (the same linears and inputs without the norms / activations in between).
    verify = None
    if not args.no_verify:
        Mv, Lv, H = 16, 36, 4096
        t0 = time.time()
        vlayers = []
        for li in range(Lv):
            g = workloads.generator(3001 + li, device=dev)
            L = [workloads.build_module(workloads.linear_spec(n, N, K, g, device=dev), dev)
                 for n, (N, K) in zip(names, shapes)]
            w_norm = (0.8 + 0.4 * torch.rand(H, generator=g, device=dev)).to(torch.bfloat16)
            vlayers.append((L, SharedInputRotateLinears(L[0:3]), SharedInputRotateLinears(L[4:6]),
                            SharedInputRotateLinears(L[6:7]), w_norm))
        torch.cuda.synchronize()
        log(f"verify block: {Lv} layers built ({time.time() - t0:.1f}s)")
        a0 = workloads.activations(Mv, H, workloads.generator(3000, device=dev), device=dev)

        def run_block(a):
            h = d = None
            for L, qkv, gu, down, w_norm in vlayers:
                if d is None:
                    q, _, _ = qkv(a)
                else:
                    # a = h + d (the previous layer's residual add) inside the q/k/v rotation launch
                    q, _, _, a = qkv(h, residual=d, return_sum=True)
                o = L[3](q)
                # h = RMSNorm(a + o) inside the gate/up group's rotation launch (also returned: next a = h + d)
                gt, up, h = gu(o, norm_weight=w_norm, eps=1e-6, residual=a, return_normed=True)
                # silu(gate) * up inside the down linear's rotation launch
                (d,) = down.forward_swiglu(gt, up)
            return h + d

        lin_in = [(a0, a0, a0, torch.nn.functional.silu(a0[:, :1].repeat(1, 3 * H)))]   # fixed inputs per layer

        def run_linears():
            xa, _, _, xd = lin_in[0]
            for L, qkv, gu, _, _ in vlayers:
                q, _, _ = qkv(xa)
                L[3](q)
                gu(xa)
                L[6](xd)

        vres = {}
        for key, fn in (("block", lambda: run_block(a0)), ("linears", run_linears)):
            fn()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                fn()
            vres[key] = time_graphs([gr], max(5, args.prefill_steps), 2)
            del gr
        vb = Lv * sum(linear_bytes(Mv, N, K) for N, K in shapes)
        verify = {"layers": Lv, "tokens": Mv, "ms_per_block": round(vres["block"], 4),
                  "linears_ms_per_block": round(vres["linears"], 4),
                  "linears_GBps": round(vb / (vres["linears"] * 1e-3) / 1e9, 1),
                  "linears_frac_hbm": round(vb / (vres["linears"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"verify block M=16 x 36 layers: {vres['block']:.3f} ms/block; quantized linears alone "
            f"{vres['linears']:.3f} ms ({verify['linears_GBps']:.0f} GB/s)")
        # The same 36-layer chain at one token: a decode step's quantized linears with the layer's
        # elementwise steps between them.  At this size the residual add and silu * mul also run inside
        # the rotation launches (the split-rotation path); "unfused" runs them as torch ops.
        a1 = workloads.activations(1, H, workloads.generator(3010, device=dev), device=dev)

        def run_block_unfused(a):
            h = d = None
            for L, qkv, gu, _, w_norm in vlayers:
                if d is not None:
                    a = h + d
                q, _, _ = qkv(a)
                o = L[3](q)
                gt, up, h = gu(o, norm_weight=w_norm, eps=1e-6, residual=a, return_normed=True)
                d = L[6](torch.nn.functional.silu(gt) * up)
            return h + d

        dres = {}
        for key, fn in (("fused", lambda: run_block(a1)), ("unfused", lambda: run_block_unfused(a1))):
            fn()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                fn()
            dres[key] = time_graphs([gr], max(5, args.prefill_steps), 2)
            del gr
        verify["decode_chain_M1"] = {"ms_per_step": round(dres["fused"], 4),
                                     "elementwise_as_torch_ops_ms": round(dres["unfused"], 4)}
        log(f"decode chain M=1 x 36 layers: {dres['fused']:.3f} ms/step; with the add and silu*mul as torch "
            f"ops {dres['unfused']:.3f} ms")
        del vlayers

    # ---- ragged packed batch: 8 requests of U{1..512} tokens ----------------
    ragged = None
    if not args.no_ragged:
        lens = workloads.ragged_lengths(8, workloads.generator(1004))
        Mr = sum(lens)
        g = workloads.generator(6100, device=dev)
        Xr = tuple(workloads.activations(Mr, K, g, device=dev) for K in (4096, 4096, 4096, 12288))
        run_layer(0, Xr, True)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            outs = run_layer(0, Xr, True)
        rms = time_graphs([gr], args.prefill_steps, 3)
        rops = sum(2 * Mr * N * K for N, K in shapes)
        ragged = {"request_tokens": lens, "total_tokens": Mr, "ms_per_layer": round(rms, 4),
                  "tops": round(rops / (rms * 1e-3) / 1e12, 1),
                  "pct_int8_peak": round(100 * rops / (rms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 2)}
        log(f"ragged batch {lens} (M={Mr}): {rms:.3f} ms/layer, {ragged['tops']:.0f} TOPS")
        del gr, outs, Xr

    # ---- W4A16 (WQLinear.forward): the same layers with fp16 activations ---
    # Each linear: rotation (fp16 result) + W4A16 GEMM (paroquant::w4a16_linear), fp16 in / out; the pool's
    # packed codes are shared, with s | sz metadata.  Decode M = 1 over the 8-layer pool (one graph), the
    # decode GEMM alone, and prefill M = 3072 (layer, GEMMs alone, each shape's GEMM alone).
    w16 = None
    if not args.no_w4a16:
        f16 = torch.float16
        w16_pool = [[(m.rotate_linear.rotation, m.rotate_linear.qlinear.qweight,
                      w16_meta(m.rotate_linear.qlinear.scales), N, K) for m, (N, K) in zip(L, shapes)]
                    for L in pool]

        def group16(members, x):
            rs = [m[0] for m in members]
            return torch.ops.paroquant.w4a16_linear_group(
                x, [r.rot_idx for r in rs], [r.rot_cs for r in rs], [r.scales_f32 for r in rs], rs[0].krot,
                [m[1] for m in members], [m[2] for m in members], [None] * len(members), False, f16)

        def run16(li, X, gemm_only=False, grouped=False):
            xa, xo, xm, xd = X
            L16 = w16_pool[li]
            if grouped:   # q/k/v and gate/up as groups over their shared inputs, o and down alone
                return (group16(L16[0:3], xa) + group16(L16[3:4], xo) + group16(L16[4:6], xm)
                        + group16(L16[6:7], xd))
            outs = []
            for (rot, wp, wm16, N, K), x in zip(L16, (xa, xa, xa, xo, xm, xm, xd)):
                if gemm_only:
                    outs.append(torch.ops.paroquant.w4a16_gemm(x, wp, wm16, None, f16))
                else:
                    outs.append(torch.ops.paroquant.w4a16_linear(x, rot.rot_idx, rot.rot_cs, rot.scales_f32,
                                                                 rot.krot, wp, wm16, None, False, f16))
            return outs

        def capture16(xs, gemm_only, layers, grouped=False):
            for li in layers:
                run16(li, xs[li], gemm_only, grouped)
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                outs = [run16(li, xs[li], gemm_only, grouped) for li in layers]
            return gr, outs

        x16 = [tuple(a.to(f16) for a in X) for X in make_inputs(1, 8001)]
        gr, _ = capture16(x16, False, range(P))
        d_ms = time_graphs([gr], -(-args.steps // P), -(-args.warmup // P)) / P
        d_b = sum(w16_linear_bytes(1, N, K) for N, K in shapes)
        del gr
        gr, _ = capture16(x16, False, range(P), grouped=True)
        dgr_ms = time_graphs([gr], -(-args.steps // P), -(-args.warmup // P)) / P
        del gr
        gr, _ = capture16(x16, True, range(P))
        dg_ms = time_graphs([gr], max(10, args.steps // 10), 3) / P
        dg_b = sum(w16_gemm_bytes(1, N, K) for N, K in shapes)
        del gr
        log(f"W4A16 decode M=1 grouped: {dgr_ms * 1e3:.1f} us/layer ({d_b / (dgr_ms * 1e-3) / 1e9:.0f} GB/s)")
        log(f"W4A16 decode M=1: {d_ms * 1e3:.1f} us/layer ({d_b / (d_ms * 1e-3) / 1e9:.0f} GB/s); GEMMs alone "
            f"{dg_ms * 1e3 / 7:.2f} us/launch ({dg_b / (dg_ms * 1e-3) / 1e9:.0f} GB/s)")
        w16 = {"decode_M1": {"us_per_layer": round(d_ms * 1e3, 2), "GBps": round(d_b / (d_ms * 1e-3) / 1e9, 1),
                             "frac_hbm": round(d_b / (d_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "gemm_only_us_per_launch": round(dg_ms * 1e3 / 7, 3),
                             "gemm_only_GBps": round(dg_b / (dg_ms * 1e-3) / 1e9, 1),
                             "gemm_only_frac_hbm": round(dg_b / (dg_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "grouped_us_per_layer": round(dgr_ms * 1e3, 2),
                             "grouped_GBps": round(d_b / (dgr_ms * 1e-3) / 1e9, 1)}}
        if not args.no_prefill:
            M = 3072
            g = workloads.generator(6200, device=dev)
            Xp = [tuple(workloads.activations(M, K, g, device=dev).to(f16) for K in (4096, 4096, 4096, 12288))]
            flops = sum(2 * M * N * K for N, K in shapes)
            pres = {}
            for gemm_only in (False, True):
                gr, outs = capture16(Xp, gemm_only, [0])
                pres[gemm_only] = time_graphs([gr], args.prefill_steps, 3)
                del gr, outs
            per_shape = {}
            xa, xo, xm, xd = Xp[0]
            for idx, x in ((0, xa), (1, xa), (4, xm), (6, xd)):
                rot, wp, wm16, N, K = w16_pool[0][idx]
                torch.ops.paroquant.w4a16_gemm(x, wp, wm16, None, f16)
                g1 = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g1):
                    for _ in range(4):
                        torch.ops.paroquant.w4a16_gemm(x, wp, wm16, None, f16)
                sms = time_graphs([g1], args.prefill_steps, 3) / 4
                per_shape[f"{N}x{K}"] = {"us": round(sms * 1e3, 1),
                                         "pct_fp16_peak": round(100 * 2 * M * N * K / (sms * 1e-3) / 1e12
                                                                / FP16_PEAK_TFLOPS, 2)}
                del g1
            lt = flops / (pres[False] * 1e-3) / 1e12
            gt = flops / (pres[True] * 1e-3) / 1e12
            w16["prefill_M3072"] = {"ms_per_layer": round(pres[False], 4), "tflops": round(lt, 1),
                                    "pct_fp16_peak": round(100 * lt / FP16_PEAK_TFLOPS, 2),
                                    "gemm_only_tflops": round(gt, 1),
                                    "gemm_only_pct_fp16_peak": round(100 * gt / FP16_PEAK_TFLOPS, 2),
                                    "gemm_per_shape": per_shape}
            log(f"W4A16 prefill M=3072: {pres[False]:.3f} ms/layer, {lt:.0f} TFLOPS ({100 * lt / FP16_PEAK_TFLOPS:.1f}%);"
                f" GEMMs alone {gt:.0f} TFLOPS; per shape " + ", ".join(f"{k} {v['us']} us ({v['pct_fp16_peak']}%)"
                                                                      for k, v in per_shape.items()))
            del Xp
        del w16_pool

    # ---- fused rotation + MXFP4 quant (rotation::rotate_and_quant_mxfp4) ----
    # bf16 activations [M, 4096] through a KROT = 8 rotation with channel scales, beside rotation::rotate
    # alone on the same input.  Bytes: x in, codes (K/2) + E8M0 scales (K/32) out, rotation parameters.
    mx = None
    if not args.no_mxfp4:
        mx = {}
        K = 4096
        g = workloads.generator(6300, device=dev)
        pairs, theta, cs = workloads.rotation_params(K, g, device=dev)
        from alpamayo_amd.quantization import Rotation
        # a prepared Rotation (bf16 buffers): the ops find its packed operands, as Rotation.forward's call does
        rot = Rotation(K, rotation_angles=theta.to(torch.bfloat16), rotation_pairs=pairs,
                       channel_scales=cs.to(torch.bfloat16)).to(dev)
        rot.prepare()
        for M in (16, 3072):
            xm = workloads.activations(M, K, g, device=dev)
            res = {}
            for name, fn in (("mxfp4", lambda: torch.ops.rotation.rotate_and_quant_mxfp4(
                                 xm, rot.pairs, rot.theta, rot.channel_scales, 128)),
                             ("rotate", lambda: rot(xm))):
                fn()
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    for _ in range(10):
                        fn()
                res[name] = time_graphs([gr], max(5, args.prefill_steps), 2) / 10
                del gr
            params = 2 * KROT * K // 2 + 2 * KROT * K + 2 * K
            b_mx = 2 * M * K + M * K // 2 + M * K // 32 + params
            b_rot = 4 * M * K + params
            mx[f"M{M}"] = {"us": round(res["mxfp4"] * 1e3, 2), "GBps": round(b_mx / (res["mxfp4"] * 1e-3) / 1e9, 1),
                           "frac_hbm": round(b_mx / (res["mxfp4"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "rotate_alone_us": round(res["rotate"] * 1e3, 2),
                           "rotate_alone_GBps": round(b_rot / (res["rotate"] * 1e-3) / 1e9, 1)}
            log(f"rotate+MXFP4 M={M} K={K}: {res['mxfp4'] * 1e3:.1f} us ({mx[f'M{M}']['GBps']:.0f} GB/s); "
                f"rotate alone {res['rotate'] * 1e3:.1f} us ({mx[f'M{M}']['rotate_alone_GBps']:.0f} GB/s)")

    # ---- rooflines ------------------------------------------------------------
    # achieved = algorithmic bytes (or int8 ops) of the launches / their time, each graph timed with HIP events
    # on its replay stream; traffic = the measured HBM bytes per launch of the same kernel (rocprofv3 counter
    # passes, profiles/), or None.
    def roof(bound, kernel, achieved_v, unit, peak, avg_us, launches, name, **extra):
        return {"bound": bound, "kernel": kernel, "achieved": round(achieved_v, 1), "peak": peak, "unit": unit,
                "frac": round(achieved_v / peak, 4), "traffic": measured_traffic(name),
                "avg_launch_us": round(avg_us, 3), "launches_timed_per_replay": launches, **extra}

    rooflines = {
        "decode_gemm_M1_layer": roof(
            "hbm", "gemm_skinny, A quantized in registers by each wave (AQ=3): the 32 GEMM launches of the "
            "8-layer pool's grouped M=1 layers (q/k/v group, o, gate/up group, down), as the headline layer runs "
            "them",
            hgemm_gbs, "GB/s", HBM_PEAK_GBS, hgemm_us, n_calls, "decode_gemm_M1_layer",
            bytes_per_launch=round(hgemm_bytes / n_calls)),
        "decode_split_rotation_M1_layer": roof(
            "hbm", "rotate_split_kernel: the 32 rotation launches of the same layers", hrot_gbs, "GB/s",
            HBM_PEAK_GBS, hrot_us, n_calls, "decode_split_rotation_M1_layer",
            bytes_per_launch=round(hrot_bytes / n_calls)),
        "decode_gemm_int8_a_M1": roof(
            "hbm", "gemm_skinny on int8 A (AQ=0), M=1: the 56 linears of the pool, one launch each",
            achieved, "GB/s", HBM_PEAK_GBS, per_launch_us, len(gemm_launches), "decode_gemm_int8_a_M1"),
    }
    if prefill is not None:
        rooflines["prefill_gemm_M3072"] = roof(
            "mfma", "gemm_prefill (tile-pair form on 192x256 / 128x256 tiles): the 7 GEMM launches of one "
            "M=3072 layer, one launch per linear", prefill["gemm_only_tops"], "TOP/s", INT8_PEAK_TOPS,
            prefill["gemm_only_ms"] * 1e3 / 7, 7, "prefill_gemm_M3072", ops_per_launch=round(prefill_ops / 7))

    # ---- CPU baseline: the oracle on the host ------------------------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)

    result = {
        "metric": "W4A8 rot+quant+GEMM: M=1 HBM GB/s; M=3072 int8 TOPS (% of peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded activations with 1% x20 outlier channels; random int4 weights, fp16 group scales)",
        "config": {
            "workload": "qwen3-8b decoder layer, 7 W4A8 linears (q,k,v,o 4096->4096/1024; gate,up 4096->12288; "
                        "down 12288->4096), decode M=1, bf16 in/out, KROT=8, group 128; q/k/v and gate/up each "
                        "run as one group over their shared input",
            "tokens_per_step": 1,
            "weight_pool_layers": args.pool_layers,
            "weight_pool_mb": round(pool_mb, 1),
            "graph_replay": True,
            "layers_per_graph": args.pool_layers,
        },
        "roofline": rooflines["decode_gemm_M1_layer"],
        "roofline_kernels": rooflines,
        "decode_gemm_per_shape_M1": gemm_per_shape,
        "decode": {f"M{M}": {"us_per_layer": round(v[0] * 1e3, 2), "GBps": round(v[1], 1),
                             "frac_hbm": round(v[1] / HBM_PEAK_GBS, 4),
                             **({"separate_linears_us_per_layer": round(decode_sep[M][0] * 1e3, 2),
                                 "separate_linears_GBps": round(decode_sep[M][1], 1)} if M in decode_sep else {})}
                   for M, v in decode.items()},
        "prefill_M3072": prefill,
        **({"library_gemms_M3072": libg} if libg is not None else {}),
        "verify_block_M16": verify,
        "ragged_batch": ragged,
        "w4a16": w16,
        "rotate_mxfp4_K4096": mx,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def cpu_cores():
    """Host cores this process may use: its affinity set, bounded by a cgroup CPU quota when one is set
    (threads beyond the quota only time-slice).  Returns (cores, affinity count, quota or None)."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = max(1, -(-int(q) // int(period)))
    except (OSError, ValueError):
        pass
    return (min(aff, quota) if quota else aff), aff, quota


def cpu_baseline(seconds: float):
    """Time the oracle's reference-path linear (AWQ unpack + dequant_awq + fp32 matmul, after the numpy rotation
    and per-token quant) on the host, on every core the process may use:
      - decode: one decoder layer's seven linears at M = 1, repeated for about `seconds` (median per layer);
      - prefill: a bounded sample of the M = 3072 layer, its q_proj-shaped linear (4096 -> 4096) at the full
        3072 rows, one pass, in int8 TOP/s (the same ops the GPU figure counts: 2*M*N*K)."""
    import numpy as np

    from alpamayo_amd import workloads
    from oracle import linear as olin
    from oracle import rotation as orot

    from threadpoolctl import threadpool_info, threadpool_limits

    cores, aff, quota = cpu_cores()

    def run(sp, c, s, x):
        return olin.reference_path_dequant(x, sp.pairs.numpy(), c, s, sp.channel_scales.float().reshape(-1).numpy(),
                                           sp.w.awq_qweight.numpy(), sp.w.awq_scales.numpy(), sp.w.awq_qzeros.numpy())

    with threadpool_limits(limits=cores):
        used = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
        specs = []
        g = workloads.generator(1001)
        for n, (N, K) in workloads.QWEN3_8B_LINEARS.items():
            sp = workloads.linear_spec(n, N, K, g)
            c, s = orot.cos_sin_table(sp.theta.numpy())
            specs.append((sp, c, s, workloads.activations(1, K, g).float().numpy()))
        layer_bytes = sum(linear_bytes(1, sp.N, sp.K) for sp, _, _, _ in specs)
        layers, t0, times = 0, time.perf_counter(), []
        while True:
            t1 = time.perf_counter()
            for sp, c, s, x in specs:
                run(sp, c, s, x)
            times.append(time.perf_counter() - t1)
            layers += 1
            if time.perf_counter() - t0 > seconds or layers >= 50:
                break
        per_layer = float(np.median(times))
        # prefill sample: the q_proj shape at M = 3072
        Mp = 3072
        sp, c, s, _ = specs[0]
        xp = workloads.activations(Mp, sp.K, workloads.generator(1010)).float().numpy()
        t1 = time.perf_counter()
        run(sp, c, s, xp)
        pf_s = time.perf_counter() - t1
    gbps = layer_bytes / per_layer / 1e9
    pf_tops = 2 * Mp * sp.N * sp.K / pf_s / 1e12
    log(f"cpu oracle: {per_layer * 1e3:.1f} ms/layer over {layers} layers, {gbps:.3f} GB/s; "
        f"M=3072 q_proj sample {pf_s:.2f} s = {pf_tops:.4f} TOP/s; {used} threads "
        f"(affinity {aff}, cgroup quota {quota})")
    return {"value": round(gbps, 4), "unit": "GB/s", "cores": int(used), "kind": "port",
            "sample": f"{layers} passes of one decoder layer's 7 linears at M=1 (median {per_layer * 1e3:.0f} "
                      "ms/layer): numpy oracle reference path (rotation, per-token int8 quant, AWQ unpack, "
                      "dequant_awq, fp32 matmul)",
            "ms_per_step": round(per_layer * 1e3, 2), "affinity_cores": aff, "cgroup_cpu_quota": quota,
            "prefill_M3072": {"value": round(pf_tops, 5), "unit": "TOP/s",
                              "pct_int8_peak": round(100 * pf_tops / INT8_PEAK_TOPS, 5),
                              "seconds": round(pf_s, 3),
                              "sample": "one pass of the layer's q_proj-shaped linear (4096->4096) at all 3072 rows "
                                        "through the same reference path (one of the M=3072 layer's 7 linears)"}}


if __name__ == "__main__":
    sys.exit(main())
