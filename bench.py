#!/usr/bin/env python3
"""Batch-1 greedy decode throughput of the Qwen3-8B-shape ternary decoder on one MI355X.

Workload (the reference's 8B decode configuration): hidden 4096, 36 layers, 32 q / 8 kv heads of
128, SwiGLU FFN 12288, vocab 151936, separate ternary LM head, fp16 KV cache to context 4096;
greedy decode of 256 tokens after a 2048-token random prompt. Weights are synthetic random
ternary (P(0) = 0.4, P(+-1) = 0.3, fp16 group scales U(0.01, 0.05)), generated in HBM by the
counter-based generator, stored as 5-trit packed rows (2-bit with --kind 2bit).

A step is one decode token: one forward of the whole model at the next position (embedding, 36
layers, LM head, on-device argmax), replayed from the captured hipGraph. The prompt is prefilled
before the clock starts (the batched prefill: `--prefill-chunk` positions per weight pass, the
last prompt position as a step), then `--warmup` tokens are decoded untimed and `--steps` tokens
timed (defaults 16 + 240 = 256 decode tokens at positions 2048..2303).

Besides the JSON contract fields the line carries
  roofline      the dominant kernel (the fused FFN gate|up GEMV with RMSNorm prologue and SwiGLU
                epilogue, 24576 x 4096) timed with HIP events on the model's stream, launched
                over the 36 resident layer matrices in turn (962 MB, more than the 256 MB
                Infinity Cache), bytes per launch = weight rows + x + norm gains + output;
  token_roofline  bytes one decode token must read (every ternary weight row, the embedding row,
                the KV cache at the mean timed position) against the same 8 TB/s;
  cpu_baseline  the float oracle's decode step (the reference's numpy CPU path restated) on a
                sample of the same shape: one layer and the LM head at context 2048, scaled to
                36 layers;
  prefill       time to first token of the prompt through the batched prefill, against the same
                prompt one position per forward (the firmware's loop), and whether both give the
                same first token;
  matvec_microbench  the isolated ternary matvec at the Qwen3-1.7B layer shapes, trit5 and 2-bit,
                over more than 512 MB of distinct matrix copies, at least 1000 matvecs per
                shape: GB/s against 8 TB/s, with the exact integer group sums checked;
  other_shapes  the same decode loop at the Qwen3-1.7B shape (256 tokens after a 512-token
                prompt) and the Qwen3.5-27B hybrid shape (128 tokens after a 1024-token prompt):
                tok/s, the bytes-per-token roofline, time to first token, and the float oracle
                timed on a sample of each shape (one layer of each kind, the LM head on a row
                sample, scaled).
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, 8 TB/s


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=None,
                    help="prompt tokens (default 2048 for the 8B shape, 1024 for the 27B hybrid)")
    ap.add_argument("--model", choices=("8b", "1.7b", "27b"), default="8b",
                    help="8b: the Qwen3-8B shape (the headline workload); 1.7b: the Qwen3-1.7B shape "
                         "(512-token prompt); 27b: the Qwen3.5-27B hybrid shape (48 Gated DeltaNet + 16 "
                         "gated attention layers); the last two report tok/s and the bytes-per-token "
                         "roofline only")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--kind", choices=("trit5", "2bit"), default="trit5")
    ap.add_argument("--kernel-reps", type=int, default=10,
                    help="passes over the 36 layers when timing the dominant kernel")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-shapes", action="store_true",
                    help="skip the Qwen3-1.7B and Qwen3.5-27B decode lines of the default run")
    ap.add_argument("--sampling", default=None, metavar="T,P,R",
                    help="sample with temperature T, top-p P and repetition penalty R instead of the "
                         "greedy argmax (the firmware's sampler; not the headline workload)")
    ap.add_argument("--no-graph", action="store_true", help="launch every kernel eagerly")
    ap.add_argument("--packed-ops", type=int, default=-1,
                    help="projections on the packed GEMV, as TRX_PACK_* bits (-1: the library's "
                         "choice for the weight kind, 0: none, 63: all)")
    ap.add_argument("--no-microbench", action="store_true",
                    help="skip the isolated matvec benchmark at the Qwen3-1.7B layer shapes")
    ap.add_argument("--only-microbench", action="store_true",
                    help="run only the isolated matvec benchmark and print its record")
    ap.add_argument("--only-kernel", action="store_true",
                    help="time only the dominant kernel (for hardware-counter runs)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="run a plain device copy of this many bytes, 10 times, and exit (the "
                         "reference kernel that calibrates the FETCH_SIZE/WRITE_SIZE counters)")
    ap.add_argument("--prefill-chunk", type=int, default=2048,
                    help="prompt positions per batched prefill forward (0: one position per forward)")
    ap.add_argument("--no-ttft-compare", action="store_true",
                    help="skip timing the one-position-per-forward prompt for comparison")
    ap.add_argument("--only-prefill", action="store_true",
                    help="time only the batched prefill of the prompt (twice) and print its record "
                         "(for kernel traces)")
    ap.add_argument("--trace-decode", type=int, default=0, metavar="N",
                    help="prefill the prompt, then run N decode positions and exit (for kernel traces "
                         "and hardware counters; with --no-graph every kernel launches eagerly)")
    ap.add_argument("--rotated", type=int, default=0, metavar="B",
                    help="a PrismML-rotated model: every projection input rotated in blocks of B columns "
                         "(the basis real Bonsai weights are stored in; 0: plain)")
    ap.add_argument("--table-free-ops", type=int, default=-1,
                    help="packed projections on the table-free lookups, as TRX_PACK_* bits (-1: the library's "
                         "choice)")
    ap.add_argument("--probes", action="store_true",
                    help="run only the streaming-read ceiling and the empty-kernel (graph node and "
                         "stream launch) probes and print their record")
    ap.add_argument("--exact-rows", type=int, default=0, metavar="N",
                    help="time the engine matvec at the 8B gate|up shape on N int8 rows in one "
                         "weight pass (trx_gemv_ternary_exact_rows) against N single-row calls, "
                         "and exit")
    return ap.parse_args()


def time_exact_rows(n, kind, reps=50):
    """The multi-row engine matvec (one weight pass for n int8 rows) against n single-row engine
    matvecs, at the Qwen3-8B gate|up shape (24576 x 4096), HIP events on one stream."""
    import ctypes
    from trixium_amd import _lib, layout as L
    from trixium_amd.bons import encode_rows
    M, K = 24576, 4096
    r = np.random.default_rng(3)
    codes = r.integers(0, 3, (M, K), dtype=np.uint8)
    scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
    rows = _lib.DeviceBuffer.from_array(encode_rows(kind, K, scales, codes))
    xs = _lib.DeviceBuffer.from_array(r.integers(-127, 128, (n, K), dtype=np.int8))
    y = _lib.DeviceBuffer(4 * n * M)
    st = _lib.DeviceBuffer(4)
    st.zero()
    B, R = 27, 24
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("trx_event_create", ctypes.byref(e0))
    _lib.call("trx_event_create", ctypes.byref(e1))

    def timed(one):
        for _ in range(5):
            one()
        _lib.call("trx_event_record", e0, None)
        for _ in range(reps):
            one()
        _lib.call("trx_event_record", e1, None)
        ms = ctypes.c_float()
        _lib.call("trx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
        return ms.value * 1e3 / reps

    def multi():
        _lib.call("trx_gemv_ternary_exact_rows", rows.ptr, kind, M, K, xs.ptr, n, B, R, y.ptr,
                  st.ptr, None)

    def singles():
        for i in range(n):
            _lib.call("trx_gemv_ternary_exact", rows.ptr, kind, M, K, xs.ptr + i * K, B, R,
                      y.ptr + 4 * i * M, st.ptr, None)

    us_multi, us_single = timed(multi), timed(singles)
    _lib.synchronize()
    _lib.call("trx_event_destroy", e0)
    _lib.call("trx_event_destroy", e1)
    wbytes = M * L.row_bytes(K, kind)
    algo = wbytes + n * K + 4 * n * M
    print(json.dumps({"kernel": "gemv_rows_kernel", "shape": [M, K], "x_rows": n,
                      "kind": "trit5" if kind == L.KIND_TERNARY5 else "2bit",
                      "us_one_pass": round(us_multi, 3), "us_single_row_calls": round(us_single, 3),
                      "speedup": round(us_single / us_multi, 2), "bytes_per_launch": algo,
                      "achieved_GBs": round(algo / (us_multi * 1e-6) / 1e9, 1), "peak_GBs": 8000,
                      "status": int(st.download(np.int32)[0])}), flush=True)


def matvec_microbench(reps=1000, rotate_bytes=512 << 20):
    """The isolated ternary matvec at the Qwen3-1.7B layer shapes (2048x2048, 1024x2048,
    6144x2048, 2048x6144), trit5 and 2-bit rows, fp16 group scales U(0.01, 0.05), P(0) = 0.4:
    y = W x with fp32 x ~ N(0, 1), batch 1. The packed GEMV runs over distinct copies of the
    matrix laid out back to back (at least `rotate_bytes` of them, more than the 256 MB Infinity
    Cache, so every launch streams from HBM), one matvec per copy in each dispatch, one x for
    all (trx_gemv_packed_batched_f32 with x_stride 0), at least two dispatches and `reps`
    matvecs timed with HIP events, queued behind one untimed dispatch so that they run back to
    back. Also timed:
    one matvec per launch (the decoder's own launch, latency bound at these sizes), and the
    engine's exact group sums on int8 x checked bit for bit against integer numpy."""
    import ctypes
    from trixium_amd import _lib, configs as C, layout as L
    from trixium_amd.bons import encode_rows
    from trixium_amd.bitexact import pack_geometry
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("trx_event_create", ctypes.byref(e0))
    _lib.call("trx_event_create", ctypes.byref(e1))

    def timed(fn, n, lead=False):
        fn()
        _lib.synchronize()
        if lead:
            # One untimed dispatch first: the GPU runs it while the host queues the timed ones,
            # so the timed dispatches run back to back (no host launch gaps between them).
            fn()
        _lib.call("trx_event_record", e0, None)
        for _ in range(n):
            fn()
        _lib.call("trx_event_record", e1, None)
        _lib.synchronize()
        ms = ctypes.c_float()
        _lib.call("trx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
        return ms.value * 1e3

    out = {}
    for M, K in C.MICROBENCH_SHAPES:
        r = np.random.default_rng(M * 7919 + K)
        u = r.random((M, K))
        codes = np.where(u < 0.3, 0, np.where(u < 0.7, 1, 2)).astype(np.uint8)
        scales = r.uniform(0.01, 0.05, (M, K // 128)).astype(np.float16)
        W64 = (codes.astype(np.float64) - 1).reshape(M, -1, 128) * scales.astype(np.float64)[:, :, None]
        W64 = W64.reshape(M, K)
        x8 = r.integers(-127, 128, K, dtype=np.int8)
        gs_want = ((codes.astype(np.int64) - 1) * x8.astype(np.int64)).reshape(M, -1, 128).sum(axis=2)
        for kind, kname in ((L.KIND_TERNARY5, "trit5"), (L.KIND_TERNARY, "2bit")):
            rows = _lib.DeviceBuffer.from_array(encode_rows(kind, K, scales, codes))
            pb, wb = pack_geometry(kind, M, K)
            stride = -(-pb // 256) * 256
            n = max(1, -(-rotate_bytes // stride))
            packed = _lib.DeviceBuffer(stride * n)
            _lib.call("trx_pack_ternary", rows.ptr, kind, M, K, 0, packed.ptr, None)
            for i in range(1, n):
                _lib.call("trx_memcpy_d2d", packed.ptr + i * stride, packed.ptr, pb, None)
            # Dispatches of n matvecs y = W x, one per copy (no two blocks read one copy, and a
            # copy is read again only a dispatch later, 512 MB on), at least `reps` in all, one x
            # for all of them (x_stride 0: a block reuses its slice's table over several matrices).
            nm = n
            x = r.standard_normal(K).astype(np.float32)
            xb = _lib.DeviceBuffer.from_array(x)
            yb = _lib.DeviceBuffer(4 * nm * M)
            bw = ctypes.c_size_t()
            _lib.call("trx_pack_batched_geometry", kind, M, K, nm, ctypes.byref(bw))
            part = _lib.DeviceBuffer(bw.value)
            _lib.synchronize()

            def batched():
                _lib.call("trx_gemv_packed_batched_f32", packed.ptr, stride, nm, n, kind, M, K, xb.ptr, 0, yb.ptr, M,
                          part.ptr, None)
            n_launch = max(2, -(-reps // n))
            us = timed(batched, n_launch, lead=True)
            # Correctness of the first and the last matvec of the dispatch (float64, 2e-6 of sum |w x|).
            y = yb.download(np.float32, nm * M).reshape(nm, M)
            err = 0.0
            ref = W64 @ x.astype(np.float64)
            mag = np.abs(W64) @ np.abs(x.astype(np.float64))
            for i in (0, nm - 1):
                err = max(err, float(np.max(np.abs(y[i] - ref) / mag)))
            row_b = L.row_bytes(K, kind)
            algo = M * row_b + 4 * K + 4 * M            # weight rows (scales + codes), fp32 x and y
            count = nm * n_launch
            gbs = algo * count / (us * 1e-6) / 1e9
            # One matvec per launch (the decoder's form), over the copies in turn.
            work = _lib.DeviceBuffer(wb)
            work.zero()
            ys = _lib.DeviceBuffer(4 * M)
            idx = [0]

            def single():
                i = idx[0] % n
                idx[0] += 1
                _lib.call("trx_gemv_packed_f32", packed.ptr + i * stride, kind, M, K, xb.ptr, None,
                          ctypes.c_float(1e-6), ys.ptr, 0, None, work.ptr, None)
            us1 = timed(single, reps) / reps
            del packed, part
            # The engine's integer matvec on int8 x (the row-packet kernel reading BONS rows as
            # stored), timed the same way: one launch over n2 copies of the rows laid back to
            # back (at least rotate_bytes, each row read once per launch), as group sums
            # gs[m][g] (the adder trees' output, G int32 per row) and as the engine-exact int32
            # result (model/bitexact.py:101-119, with the tensor's B and R). The first and last
            # copies' group sums are checked bit for bit against integer numpy, and their exact
            # results against one launch over a single copy.
            G = K // 128
            row_b = L.row_bytes(K, kind)
            mat_b = M * row_b
            n2 = max(1, -(-rotate_bytes // mat_b))
            rot = _lib.DeviceBuffer(mat_b * n2)
            for i in range(n2):
                _lib.call("trx_memcpy_d2d", rot.ptr + i * mat_b, rows.ptr, mat_b, None)
            xq = _lib.DeviceBuffer.from_array(x8)
            gsb = _lib.DeviceBuffer(4 * n2 * M * G)
            n_int = max(2, -(-reps // n2))
            us_gs = timed(lambda: _lib.call("trx_gemv_ternary_groupsums", rot.ptr, kind, n2 * M, K, xq.ptr, gsb.ptr,
                                            None), n_int, lead=True)
            gs = gsb.download(np.int32, n2 * M * G).reshape(n2, M, G)
            gs_ok = bool(np.array_equal(gs[0], gs_want) and np.array_equal(gs[-1], gs_want))
            del gsb
            B_, R_ = exact_scale_bias(scales)
            yb_ex = _lib.DeviceBuffer(4 * n2 * M)
            st = _lib.DeviceBuffer(4)
            st.zero()
            us_ex = timed(lambda: _lib.call("trx_gemv_ternary_exact", rot.ptr, kind, n2 * M, K, xq.ptr, B_, R_,
                                            yb_ex.ptr, st.ptr, None), n_int, lead=True)
            y1 = _lib.DeviceBuffer(4 * M)
            _lib.call("trx_gemv_ternary_exact", rows.ptr, kind, M, K, xq.ptr, B_, R_, y1.ptr, st.ptr, None)
            _lib.synchronize()
            ex = yb_ex.download(np.int32, n2 * M).reshape(n2, M)
            one = y1.download(np.int32, M)
            ex_ok = bool(np.array_equal(ex[0], one) and np.array_equal(ex[-1], one)
                         and st.download(np.int32, 1)[0] == 0)
            gs_bytes = mat_b + K + 4 * M * G            # rows, int8 x, int32 group sums
            ex_bytes = mat_b + K + 4 * M
            gs_gbs = gs_bytes * n2 * n_int / (us_gs * 1e-6) / 1e9
            ex_gbs = ex_bytes * n2 * n_int / (us_ex * 1e-6) / 1e9
            del rot, yb_ex
            out[f"{M}x{K}/{kname}"] = {
                "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "us_per_matvec": round(us / count, 3),
                "bytes_per_matvec": algo, "matvecs": count, "copies": n, "rotated_MB": round(n * stride / 2**20, 1),
                "single_launch_us": round(us1, 3), "single_launch_GBs": round(algo / (us1 * 1e-6) / 1e9, 1),
                "max_rel_err": float(f"{err:.2e}"),
                "exact_int8": {"groupsums_GBs": round(gs_gbs, 1), "groupsums_frac": round(gs_gbs / HBM_PEAK_GBS, 4),
                               "groupsums_bytes_per_matvec": gs_bytes, "groupsums_bitexact": gs_ok,
                               "engine_exact_GBs": round(ex_gbs, 1), "engine_exact_frac": round(ex_gbs / HBM_PEAK_GBS, 4),
                               "engine_exact_bytes_per_matvec": ex_bytes, "engine_exact_equal": ex_ok,
                               "matvecs": n2 * n_int}}
            del xb, yb, rows
    _lib.call("trx_event_destroy", e0)
    _lib.call("trx_event_destroy", e1)
    tot_bytes = sum(v["bytes_per_matvec"] * v["matvecs"] for v in out.values())
    tot_us = sum(v["us_per_matvec"] * v["matvecs"] for v in out.values())
    agg = tot_bytes / (tot_us * 1e-6) / 1e9
    gs_b = sum(v["exact_int8"]["groupsums_bytes_per_matvec"] * v["exact_int8"]["matvecs"] for v in out.values())
    gs_t = sum(v["exact_int8"]["groupsums_bytes_per_matvec"] * v["exact_int8"]["matvecs"] / v["exact_int8"]["groupsums_GBs"]
               for v in out.values())
    return {"kernel": "packed table-lookup GEMV, many matvecs y = W x per dispatch over rotating copies of W "
                      "(trx_gemv_packed_batched_f32, one x: each block reuses its slice's table over several "
                      "matrices), fp32 x and y", "aggregate_GBs": round(agg, 1), "aggregate_frac": round(agg / HBM_PEAK_GBS, 4),
            "exact_int8_kernel": "row-packet engine kernel on int8 x over BONS rows as stored "
                                 "(trx_gemv_ternary_groupsums / trx_gemv_ternary_exact), one launch over the copies",
            "exact_int8_groupsums_aggregate_GBs": round(gs_b / gs_t, 1),
            "peak_GBs": HBM_PEAK_GBS, "shapes": out}


def exact_scale_bias(scales):
    """The engine's per-tensor B and R for fp16 scales (model/bitexact.py:56-97):
    B = 12 - max exponent, R the smallest shift that keeps every result within int32."""
    from trixium_amd.fixedpoint import scale_bias, result_shift
    B = scale_bias(scales)
    return B, result_shift(scales, B)


def copy_calibration(nbytes):
    """A device-to-device copy kernel of known size (torch's elementwise copy)."""
    import torch
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "launches": 10}), flush=True)


def time_dominant_kernel(dec, mc, reps, graph=True):
    """Average duration of the gate|up GEMV over the resident layer matrices (HIP events on the
    model stream), launched as the decode launches it: with the packed gate|up and down, the
    partial sums and slice sums of x^2 that down's prologue reduces. graph: the 36 launches are
    captured into one hipGraph and replayed `reps` times, as the decode's graph replays its
    kernels back to back (otherwise eager launches, for kernel traces)."""
    import ctypes
    from trixium_amd import _lib, layout as L
    from trixium_amd.model import PACK_GATE_UP, PACK_DOWN
    E, F = mc.n_embd, mc.ffn_dim
    x = _lib.DeviceBuffer.from_array(np.random.default_rng(1).standard_normal(E).astype(np.float32))
    y = _lib.DeviceBuffer(F * 4)
    s = dec.stream
    kind = dec.cfg.weight_kind
    norms = [dec.tensor_ptr(L.ROLE_FFN_NORM, l)[0] for l in range(mc.n_layer)]
    mode = "row-packet"
    if dec.packed_ops & PACK_GATE_UP:
        mats = [dec.packed_ptr(PACK_GATE_UP, l) for l in range(mc.n_layer)]
        mode = "packed partials" if dec.packed_ops & PACK_DOWN else "packed"
        if mode == "packed partials":
            S, rp, bps = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
            _lib.call("trx_pack_partials_geometry", kind, 2 * F, E, ctypes.byref(S), ctypes.byref(rp), ctypes.byref(bps))
            part = _lib.DeviceBuffer(4 * S.value * rp.value)
            ss = _lib.DeviceBuffer(4 * S.value * bps.value)
            parts = _lib.PartialSums(out=part.ptr, out_ss=ss.ptr)

            def launch():
                for (w, ws), g in zip(mats, norms):
                    _lib.call("trx_gemv_packed_parts_f32", w, kind, 2 * F, E, x.ptr, g, ctypes.c_float(mc.rms_eps),
                              None, _lib.EPI_SWIGLU, None, ws, ctypes.byref(parts), s)
        else:
            def launch():
                for (w, ws), g in zip(mats, norms):
                    _lib.call("trx_gemv_packed_f32", w, kind, 2 * F, E, x.ptr, g, ctypes.c_float(mc.rms_eps),
                              y.ptr, _lib.EPI_SWIGLU, None, ws, s)
    else:
        mats = [dec.tensor_ptr(L.ROLE_FFN_GATE, l)[0] for l in range(mc.n_layer)]

        def launch():
            for w, g in zip(mats, norms):
                _lib.call("trx_gemv_ternary_f32", w, kind, 2 * F, E, x.ptr, g, ctypes.c_float(mc.rms_eps),
                          y.ptr, _lib.EPI_SWIGLU, None, s)

    launch()
    _lib.call("trx_stream_sync", s)
    run = launch
    exe = None
    if graph:
        exe = ctypes.c_void_p()
        _lib.call("trx_graph_begin", s)
        launch()
        _lib.call("trx_graph_end", s, ctypes.byref(exe))

        def run():
            _lib.call("trx_graph_launch", exe, s)
        run()
        _lib.call("trx_stream_sync", s)
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("trx_event_create", ctypes.byref(e0))
    _lib.call("trx_event_create", ctypes.byref(e1))
    _lib.call("trx_event_record", e0, s)
    for _ in range(reps):
        run()
    _lib.call("trx_event_record", e1, s)
    _lib.call("trx_stream_sync", s)
    if exe is not None:
        _lib.call("trx_graph_destroy", exe)
    ms = ctypes.c_float()
    _lib.call("trx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
    _lib.call("trx_event_destroy", e0)
    _lib.call("trx_event_destroy", e1)
    n = reps * len(mats)
    rb = L.row_bytes(E, kind)
    algo = 2 * F * rb + E * 4 + E * 4 + F * 4
    return ms.value * 1e3 / n, algo, n, mode


def probes(read_bytes=1 << 30, nodes=400, reps=10):
    """Two references the kernels are held to, measured on this GPU: a plain streaming read of
    device memory (trx_probe_stream_read over read_bytes, the best of a few launch shapes: the
    practical read ceiling, against the 8 TB/s peak), and the fixed cost of an empty kernel as a
    dependent node of a replayed hipGraph and as a stream launch (trx_probe_empty)."""
    import ctypes
    from trixium_amd import _lib
    s = ctypes.c_void_p()
    _lib.call("trx_stream_create", ctypes.byref(s))
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("trx_event_create", ctypes.byref(e0))
    _lib.call("trx_event_create", ctypes.byref(e1))

    def timed(fn, n):
        fn()
        _lib.call("trx_stream_sync", s)
        _lib.call("trx_event_record", e0, s)
        for _ in range(n):
            fn()
        _lib.call("trx_event_record", e1, s)
        _lib.call("trx_stream_sync", s)
        ms = ctypes.c_float()
        _lib.call("trx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
        return ms.value * 1e3 / n

    buf = _lib.DeviceBuffer(read_bytes)
    buf.zero()
    out = _lib.DeviceBuffer(4 * 4096)
    shapes = {}
    for blocks, threads in ((256, 1024), (512, 1024), (1024, 512), (2048, 256), (4096, 256)):
        us = timed(lambda: _lib.call("trx_probe_stream_read", buf.ptr, read_bytes, out.ptr, blocks, threads, s), 10)
        shapes[f"{blocks}x{threads}"] = round(read_bytes / (us * 1e-6) / 1e9, 1)
    best = max(shapes.values())
    del buf
    stream_us = timed(lambda: _lib.call("trx_probe_empty", s), 2000)
    exe = ctypes.c_void_p()
    _lib.call("trx_graph_begin", s)
    for _ in range(nodes):
        _lib.call("trx_probe_empty", s)
    _lib.call("trx_graph_end", s, ctypes.byref(exe))
    node_us = timed(lambda: _lib.call("trx_graph_launch", exe, s), reps) / nodes
    _lib.call("trx_graph_destroy", exe)
    _lib.call("trx_event_destroy", e0)
    _lib.call("trx_event_destroy", e1)
    _lib.call("trx_stream_destroy", s)
    return {"stream_read": {"GBs": best, "frac_of_peak": round(best / HBM_PEAK_GBS, 4), "bytes": read_bytes,
                            "by_blocks_x_threads": shapes},
            "empty_kernel_us": {"graph_node": round(node_us, 3), "stream_launch": round(stream_us, 3),
                                "graph_nodes": nodes}}


def traffic_from_profile(kind, mode):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 counter summary
    (FETCH_SIZE + WRITE_SIZE, calibrated on a copy kernel), when one exists for this format and
    kernel."""
    tag = {"row-packet": "", "packed": "_packed", "packed partials": "_packed_partials"}[mode]
    path = os.path.join(ROOT, "profiles", f"gemv_gateup_8b_{kind}{tag}_pmc.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def blas_info():
    """numpy's BLAS library and version, as numpy reports them."""
    try:
        cfg = np.show_config(mode="dicts")
        b = cfg.get("Build Dependencies", {}).get("blas", {})
        return f"{b.get('name', '?')} {b.get('version', '')}".strip()
    except Exception:
        return "unknown"


def tiny_cpu_decode(seed=0, n_prompt=16, n_new=64):
    """The tiny random Qwen3 model (hidden 256, 4 layers, vocab 2048, seed 0): the float oracle's
    full greedy decode of 64 tokens after a 16-token prompt, timed on the host, and the GPU
    decoder's tokens for the same model and prompt."""
    import tempfile
    from oracle.floatref import FloatRef
    from trixium_amd import bons, configs as C, synth
    from trixium_amd.model import Decoder
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.img")
        bons.write_image(C.TINY, synth.small_model_tensors(C.TINY, seed, True), 1, path, trit5=True)
        prompt = synth.random_prompt(C.TINY, n_prompt, seed)
        ref = FloatRef(bons.BONSReader(path), kv_fp16=True)
        t0 = time.perf_counter()
        cpu = ref.generate(prompt, n_new)
        dt = time.perf_counter() - t0
        dec = Decoder.from_image(path, max_new=n_new)
        gpu = dec.generate_fresh(prompt, n_new)
        dec.close()
    return {"config": "tiny qwen3 (256 wide, 4 layers, vocab 2048), seed 0", "prompt_tokens": n_prompt,
            "new_tokens": n_new, "seconds": round(dt, 3), "tok_s": round(n_new / dt, 2),
            "tokens_equal_gpu": cpu == gpu}


def cpu_baseline(mc, ctx):
    """The oracle's decode step on one layer + the LM head of the shape, scaled to all layers;
    and the tiny model's full greedy decode."""
    from oracle.floatref import ShapeSample
    cores = len(os.sched_getaffinity(0))
    threads = int(os.environ.get("OMP_NUM_THREADS", cores))
    s = ShapeSample(mc, 1, ctx, seed=0)
    s.step(1)                                   # first touch of every buffer
    t0 = time.perf_counter()
    s.step(2, want_logits=False)
    t_layer = time.perf_counter() - t0
    t0 = time.perf_counter()
    s.step(3, want_logits=True)
    t_head = max(time.perf_counter() - t0 - t_layer, 0.0)
    per_tok = mc.n_layer * t_layer + t_head
    tiny = tiny_cpu_decode()
    return {"value": round(1.0 / per_tok, 6), "unit": "tok/s", "cores": min(cores, threads),
            "blas": blas_info(), "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "tiny_decode": tiny,
            "kind": "port",
            "sample": (f"float oracle decode step (numpy, fp16 weight cache) on 1 of {mc.n_layer} "
                       f"layers + the {mc.vocab}x{mc.n_embd} LM head at context {ctx}: "
                       f"layer {t_layer:.2f} s, head {t_head:.2f} s, token = {mc.n_layer} x layer + head "
                       f"= {per_tok:.1f} s")}


def cpu_shape_sample(mc, ctx, head_rows=16384):
    """The float oracle's decode step at a shape, timed on a sample: one layer of each kind the
    model has (full size, context ctx) and the LM head over head_rows of its rows, scaled to the
    model's layer counts and vocabulary (a matvec's time is linear in its rows)."""
    import dataclasses
    from oracle.floatref import ShapeSample
    small = dataclasses.replace(mc, vocab=head_rows)
    kinds = ["attn"] + (["deltanet"] if mc.n_dn_layers else [])
    per_kind, t_head = {}, []
    for k in kinds:
        s = ShapeSample(small, 1, ctx, seed=0, kinds=[k])
        s.step(1)                               # first touch of every buffer
        t0 = time.perf_counter()
        s.step(2, want_logits=False)
        per_kind[k] = time.perf_counter() - t0
        t0 = time.perf_counter()
        s.step(3, want_logits=True)
        t_head.append(max(time.perf_counter() - t0 - per_kind[k], 0.0))
        del s
    head = min(t_head) * mc.vocab / head_rows
    n_dn = mc.n_dn_layers
    per_tok = (mc.n_layer - n_dn) * per_kind["attn"] + n_dn * per_kind.get("deltanet", 0.0) + head
    layers = " + ".join(f"{n} x {k} layer {per_kind[k]:.2f} s" for k, n in
                        (("attn", mc.n_layer - n_dn), ("deltanet", n_dn)) if n)
    cores = len(os.sched_getaffinity(0))
    threads = int(os.environ.get("OMP_NUM_THREADS", cores))
    return {"value": round(1.0 / per_tok, 6), "unit": "tok/s", "cores": min(cores, threads), "kind": "port",
            "sample": (f"float oracle decode step (numpy, fp16 weight cache) at context {ctx}: one layer of "
                       f"each kind and the LM head over {head_rows} of its {mc.vocab} rows, scaled: "
                       f"{layers} + head {head:.2f} s = {per_tok:.1f} s per token")}


def decode_at_shape(mc, prompt_len, n_dec, warmup, seed, kind, graph=True, packed_ops=-1, table_free_ops=-1,
                    rotated=0, sampling=None, prefill_chunk=2048):
    """Batch-1 decode of a synthetic model of shape mc: time to first token of a random prompt
    through the batched prefill, then `warmup` untimed and n_dec - warmup timed decode tokens
    (hipGraph replay). Returns (tok/s, seconds timed, record, decoder)."""
    from trixium_amd import layout as L
    from trixium_amd.model import Decoder, INFO_WEIGHT_BYTES
    dec = Decoder.synthetic(mc, seed, weight_kind=kind, max_ctx=mc.max_ctx, max_new=n_dec + 8,
                            use_graph=graph, packed_ops=packed_ops, table_free_ops=table_free_ops,
                            hadamard_block=rotated)
    prompt = np.random.default_rng(seed).integers(0, mc.vocab, prompt_len).astype(np.int32)
    if sampling:
        t, p_, r = (float(v) for v in sampling.split(","))
        dec.set_sampling(t, p_, r, seed=seed + 1)
    ttft = []
    for _ in range(2):
        dec.reset()
        dec.feed(prompt)
        dec.synchronize()
        t0 = time.perf_counter()
        dec.prefill(prompt_len - 1, prefill_chunk)
        dec.step(1)
        dec.synchronize()
        ttft.append(time.perf_counter() - t0)
    dec.step(warmup)
    dec.synchronize()
    steps = n_dec - 1 - warmup
    t0 = time.perf_counter()
    dec.step(steps)
    dec.synchronize()
    dt = time.perf_counter() - t0
    dec.finalize()
    toks = dec.outputs()[:n_dec]
    assert np.all((toks >= 0) & (toks < mc.vocab)), "decoded ids out of range"
    tok_s = steps / dt
    # Bytes per token: the weights (a tied head reads the whole embedding table, an untied model
    # one embedding row), K/V of the attention layers up to the mean timed position, every
    # DeltaNet layer's recurrent state read and written.
    wbytes = dec.info(INFO_WEIGHT_BYTES)
    emb_rows = dec.tensor_ptr(L.ROLE_TOK_EMB, 0)[1]
    emb_row = L.row_bytes(mc.n_embd, kind)
    mean_pos = prompt_len + warmup + (steps - 1) / 2.0
    n_attn = mc.n_layer - mc.n_dn_layers
    kv = 2 * n_attn * mc.n_kv_head * mc.head_dim * 2 * (mean_pos + 1)
    dn = 2 * mc.n_dn_layers * mc.dn_num_v_heads * mc.dn_v_head_dim * mc.dn_k_head_dim * 4
    tok_bytes = wbytes + (0 if mc.tie_embeddings else emb_row - emb_rows) + kv + dn
    roof = HBM_PEAK_GBS * 1e9 / tok_bytes
    rec = {"prompt_tokens": prompt_len, "decode_tokens": n_dec, "timed_tokens": steps,
           "tok_s": round(tok_s, 2), "ms_per_token": round(1e3 / tok_s, 4),
           "token_roofline": {"bytes_per_token": int(tok_bytes), "tok_s": round(roof, 1),
                              "frac": round(tok_s / roof, 4)},
           "ttft_ms": round(min(ttft) * 1e3, 2), "prefill_chunk": prefill_chunk,
           "packed_ops": dec.packed_ops}
    return tok_s, dt, rec, dec


# The other decode workloads: the Qwen3-1.7B shape (256 tokens after a 512-token prompt) and the
# Qwen3.5-27B hybrid shape (128 tokens after a 1024-token prompt).
OTHER_SHAPES = (("1.7b", 512, 256), ("27b", 1024, 128))


def other_shapes(kind, seed, cpu=True):
    from trixium_amd import configs as C
    out = {}
    for key, prompt_len, n_dec in OTHER_SHAPES:
        mc = {"1.7b": C.QWEN3_1P7B, "27b": C.QWEN35_27B}[key]
        _, _, rec, dec = decode_at_shape(mc, prompt_len, n_dec, 16, seed, kind)
        dec.close()
        if cpu:
            rec["cpu_baseline"] = cpu_shape_sample(mc, prompt_len)
        out[mc.name] = rec
    return out


def main():
    a = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the batch-1 decode loop runs on a single MI355X "
              f"(asked for {max(a.gpus, world)}); run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if a.copy_bytes:
        copy_calibration(a.copy_bytes)
        return
    from trixium_amd import configs as C, layout as L, _lib
    from trixium_amd.model import Decoder, INFO_WEIGHT_BYTES
    if a.exact_rows:
        time_exact_rows(a.exact_rows, L.KIND_TERNARY5 if a.kind == "trit5" else L.KIND_TERNARY)
        return
    if a.only_microbench:
        print(json.dumps({"matvec_microbench": matvec_microbench()}), flush=True)
        return
    if a.probes:
        print(json.dumps({"probes": probes()}), flush=True)
        return
    mc = {"8b": C.QWEN3_8B, "1.7b": C.QWEN3_1P7B, "27b": C.QWEN35_27B}[a.model]
    if a.prompt is None:
        a.prompt = {"8b": 2048, "1.7b": 512, "27b": 1024}[a.model]
    kind = L.KIND_TERNARY5 if a.kind == "trit5" else L.KIND_TERNARY
    if a.only_kernel:
        dec = Decoder.synthetic(mc, a.seed, weight_kind=kind, max_ctx=mc.max_ctx, max_new=8,
                                packed_ops=a.packed_ops, table_free_ops=a.table_free_ops,
                                hadamard_block=a.rotated)
        us, algo, n_launch, _ = time_dominant_kernel(dec, mc, a.kernel_reps, graph=not a.no_graph)
        print(json.dumps({"kernel_us": round(us, 3), "bytes_per_launch": algo, "launches": n_launch,
                          "timing": "eager launches" if a.no_graph else "graph replay",
                          "achieved_GBs": round(algo / (us * 1e-6) / 1e9, 1)}), flush=True)
        dec.close()
        return
    if a.only_prefill or a.trace_decode:
        dec = Decoder.synthetic(mc, a.seed, weight_kind=kind, max_ctx=mc.max_ctx, max_new=a.trace_decode + 8,
                                use_graph=not a.no_graph, packed_ops=a.packed_ops, table_free_ops=a.table_free_ops,
                                hadamard_block=a.rotated)
        prompt = np.random.default_rng(a.seed).integers(0, mc.vocab, a.prompt).astype(np.int32)
        chunk = a.prefill_chunk or 2048
        for rep in range(2 if a.only_prefill else 1):
            dec.reset()
            dec.feed(prompt)
            dec.synchronize()
            t0 = time.perf_counter()
            dec.prefill(a.prompt - 1, chunk)
            dec.step(1)
            dec.synchronize()
            print(json.dumps({"prefill_rep": rep, "prompt_tokens": a.prompt, "chunk": chunk,
                              "ttft_ms": round((time.perf_counter() - t0) * 1e3, 2)}), flush=True)
        if a.trace_decode:
            dec.step(a.trace_decode)
            dec.synchronize()
            print(json.dumps({"decode_positions": a.trace_decode}), flush=True)
        dec.close()
        return
    n_dec = a.warmup + a.steps
    if a.prompt + n_dec > mc.max_ctx:
        sys.exit(f"prompt {a.prompt} + {n_dec} decode tokens exceed the context {mc.max_ctx}")
    graph = not a.no_graph
    if a.model != "8b":
        tok_s, dt, rec, dec = decode_at_shape(mc, a.prompt, 1 + n_dec, a.warmup, a.seed, kind, graph, a.packed_ops,
                                              a.table_free_ops, a.rotated, a.sampling, a.prefill_chunk or 2048)
        print(json.dumps({
            "metric": f"batch-1 decode tok/s ({mc.name})", "value": rec["tok_s"], "unit": "tok/s",
            "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": rec["ms_per_token"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "ternary weights (fp16 group scales), fp32 activations, fp32 accumulate, fp16 KV"
                     + (", fp32 DeltaNet state" if mc.n_dn_layers else ""),
            "data": "synthetic: random ternary weights from a counter-based hash, random prompt",
            "config": {"workload": f"{mc.name} ternary decoder, batch-1 greedy decode after a "
                                   f"{a.prompt}-token prompt", "n_layer": mc.n_layer, "n_embd": mc.n_embd,
                       "ffn_dim": mc.ffn_dim, "vocab": mc.vocab, "prompt_tokens": a.prompt,
                       "decode_tokens": 1 + n_dec, "weights": a.kind, "hipgraph": graph,
                       "packed_ops": dec.packed_ops, "table_free_ops": dec.table_free_ops,
                       "rotation_block": a.rotated},
            "token_roofline": rec["token_roofline"], "roofline": None,
            "cpu_baseline": None if a.no_cpu_baseline else cpu_shape_sample(mc, a.prompt),
            "prefill": {"prompt_tokens": a.prompt, "chunk": rec["prefill_chunk"], "ttft_ms": rec["ttft_ms"]}}),
            flush=True)
        dec.close()
        return
    dec = Decoder.synthetic(mc, a.seed, weight_kind=kind, max_ctx=mc.max_ctx, max_new=n_dec + 8,
                            use_graph=graph, packed_ops=a.packed_ops, table_free_ops=a.table_free_ops,
                                hadamard_block=a.rotated)
    prompt = np.random.default_rng(a.seed).integers(0, mc.vocab, a.prompt).astype(np.int32)
    if a.sampling:
        t, p_, r = (float(v) for v in a.sampling.split(","))
        dec.set_sampling(t, p_, r, seed=a.seed + 1)
    # Time to first token: the prompt's first a.prompt - 1 positions through the batched prefill
    # (a.prefill_chunk positions per weight pass), then the last prompt position, whose forward
    # computes the logits and the first generated token. For comparison, the same prompt one
    # position per forward (the firmware's loop); both give the same first token.
    prefill = None
    if a.prefill_chunk > 0:
        ttft = []
        for _ in range(2):
            dec.reset()
            dec.feed(prompt)
            dec.synchronize()
            t0 = time.perf_counter()
            dec.prefill(a.prompt - 1, a.prefill_chunk)
            dec.step(1)
            dec.synchronize()
            ttft.append(time.perf_counter() - t0)
        dec.finalize()
        first = int(dec.outputs()[0])
        prefill = {"prompt_tokens": a.prompt, "chunk": a.prefill_chunk, "ttft_ms": round(min(ttft) * 1e3, 2),
                   "prompt_tok_s": round(a.prompt / min(ttft), 1)}
        if not a.no_ttft_compare:
            dec.reset()
            dec.feed(prompt)
            dec.synchronize()
            t0 = time.perf_counter()
            dec.step(a.prompt)
            dec.synchronize()
            t1 = time.perf_counter() - t0
            dec.finalize()
            prefill.update({"ttft_ms_one_position_per_forward": round(t1 * 1e3, 2),
                            "speedup": round(t1 / min(ttft), 2),
                            "first_token_match": int(dec.outputs()[0]) == first})
    dec.reset()
    dec.feed(prompt)
    if a.prefill_chunk > 0:
        dec.prefill(a.prompt - 1, a.prefill_chunk)
        dec.step(1)
    else:
        dec.step(a.prompt)                       # one position per forward
    dec.synchronize()
    dec.step(a.warmup)
    dec.synchronize()
    t0 = time.perf_counter()
    dec.step(a.steps)
    dec.synchronize()
    dt = time.perf_counter() - t0
    tok_s = a.steps / dt
    dec.finalize()
    toks = dec.outputs()[:n_dec]
    assert np.all((toks >= 0) & (toks < mc.vocab)), "decoded ids out of range"

    # Bytes per decode token: every weight row except the embedding table, which is read one
    # row per token; the K and V caches up to the mean timed position.
    wbytes = dec.info(INFO_WEIGHT_BYTES)
    emb_rows = dec.tensor_ptr(L.ROLE_TOK_EMB, 0)[1]
    emb_row = L.row_bytes(mc.n_embd, kind)
    mean_pos = a.prompt + a.warmup + (a.steps - 1) / 2.0
    kv = 2 * mc.n_layer * mc.n_kv_head * mc.head_dim * 2 * (mean_pos + 1)
    tok_bytes = wbytes - emb_rows + emb_row + kv
    roof_tok_s = HBM_PEAK_GBS * 1e9 / tok_bytes


    us, algo, n_launch, gu_mode = time_dominant_kernel(dec, mc, a.kernel_reps, graph=graph)
    achieved = algo / (us * 1e-6) / 1e9
    from trixium_amd.model import PACK_QKV, PACK_O, PACK_GATE_UP, PACK_DOWN
    layer_ops = PACK_QKV | PACK_O | PACK_GATE_UP | PACK_DOWN
    acts = ("fp32 activations" if dec.packed_ops & layer_ops == layer_ops
            else "fp32 activations (packed GEMV) / int16 per 128-group (row-packet GEMV)")
    kdesc = {"packed partials": "RMSNorm fused (its scale applied by the consumer), split-K partial sums "
                                "handed to down's prologue (SwiGLU there), packed table-lookup kernel",
             "packed": "RMSNorm + SwiGLU fused, packed table-lookup kernel",
             "row-packet": "RMSNorm + SwiGLU fused, row-packet kernel"}[gu_mode]
    rec = {
        "metric": "batch-1 decode tok/s (8B shape); ternary matvec HBM GB/s vs ~8 TB/s peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dt * 1e3 / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"ternary weights (fp16 group scales), {acts}, fp32 accumulate, fp16 KV",
        "data": "synthetic: random ternary weights from a counter-based hash, random prompt",
        "config": {"workload": "qwen3-8b-shape ternary decoder, batch-1 "
                               + (f"sampled (T,P,R={a.sampling})" if a.sampling else "greedy")
                               + f" decode after a {a.prompt}-token prompt",
                   "n_layer": mc.n_layer, "n_embd": mc.n_embd, "n_head": mc.n_head,
                   "n_kv_head": mc.n_kv_head, "head_dim": mc.head_dim, "ffn_dim": mc.ffn_dim,
                   "vocab": mc.vocab, "max_ctx": mc.max_ctx, "prompt_tokens": a.prompt,
                   "decode_tokens": n_dec, "weights": a.kind, "hipgraph": graph,
                   "packed_ops": dec.packed_ops, "table_free_ops": dec.table_free_ops,
                   "rotation_block": a.rotated},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile(a.kind, gu_mode),
                     "kernel": f"ternary GEMV gate|up {2 * mc.ffn_dim}x{mc.n_embd} {a.kind}, {kdesc}",
                     "us_per_launch": round(us, 3), "bytes_per_launch": algo, "launches": n_launch,
                     "timing": ("HIP events over replays of a hipGraph of the 36 layers' launches (the decode's "
                                "form)" if graph else "HIP events over eager launches")},
        "token_roofline": {"bytes_per_token": int(tok_bytes), "tok_s": round(roof_tok_s, 1),
                           "frac": round(tok_s / roof_tok_s, 4)},
        "cpu_baseline": None,
        "prefill": prefill,
    }
    dec.close()
    rec["probes"] = probes()
    if not a.no_microbench:
        rec["matvec_microbench"] = matvec_microbench()
    if not a.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline(mc, a.prompt)
    if not a.no_other_shapes:
        rec["other_shapes"] = other_shapes(kind, a.seed, cpu=not a.no_cpu_baseline)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
