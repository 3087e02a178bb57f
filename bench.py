"""Regrow benchmark: bit-exact requantization of BF16 weights (with the imatrix) on one MI355X.

A step is one pass of the hot path over one batch of synthetic input: the configuration-2 workload
-- the K-quant family Q2_K, Q3_K, Q4_K, Q5_K, Q6_K with an imatrix, on
the two Qwen3-0.6B-shaped BF16 tensors token_embd 151936x1024 and ffn_down 1024x3072 (10 launches
per step, inputs resident in HBM before timing starts).

value = BF16 bytes consumed per step / step time (GB/s), i.e. the requant throughput of the family.
Per-type throughput, the HBM-bound legacy types (Q8_0 / Q4_0 on configuration 1 and on the
embedding) and the reference's own C quantizers on the host cores (cpu_baseline) are reported in the
same JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import collections
import concurrent.futures
import json
import os
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
KTYPES = [10, 11, 12, 13, 14]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def alg_bytes(t, nw, npr, imx):
    """algorithmic HBM bytes of one requant launch: BF16 in + quant out + imatrix"""
    from seedpack_amd.requant import QFUN
    _, qk, bs = QFUN[t]
    return 2 * nw + nw // qk * bs + (4 * npr if imx else 0)


def _timed_sample(run, x, budget_s):
    """run(rows) on a row sample of x sized so that it takes about budget_s (measured on 1/16 of the
    rows first) -> (rows, seconds)"""
    probe = max(1, x.shape[0] // 16)
    t0 = time.perf_counter()
    run(x[:probe])
    per_row = (time.perf_counter() - t0) / probe
    rows = int(min(x.shape[0], max(probe, budget_s / max(per_row, 1e-9))))
    t0 = time.perf_counter()
    run(x[:rows])
    return rows, time.perf_counter() - t0


def cpu_baseline(tensors, target_s=12.0, type_s=1.5):
    """the reference's C quantizers (oracle/_ref) on the host cores: the configuration-2 family on the
    first rows of the embedding (the line's figure, a bounded sample of the same workload), then per
    type on a bounded row sample of its own configuration's tensor (Q8_0 / Q4_0: configuration 1 without
    imatrix; the K-quants: the embedding with its imatrix; the i-quants: the configuration-3
    4096x12288 Student-t tensor with its imatrix); and the QR encoder of configuration 1 as the
    oracle's single-core numpy port (oracle/qr.py)"""
    from oracle import qr as oqr
    from oracle import ref
    from seedpack_amd import synth
    from seedpack_amd.requant import NAMES
    if not ref.available():
        return None
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    (w_emb, imx_emb) = tensors["token_embd"]
    (w_dn, imx_dn) = tensors["ffn_down"]
    x = synth.bf16_to_f32(w_dn).reshape(w_dn.shape)
    t0 = time.perf_counter()
    for t in KTYPES:
        ref.quantize(t, x, imx_dn, threads=threads)
    rate = 5 * x.size / (time.perf_counter() - t0)             # weights/s over the family
    rows = int(min(w_emb.shape[0], max(1024, target_s * rate / 5 / w_emb.shape[1])))
    xe = synth.bf16_to_f32(w_emb[:rows]).reshape(rows, w_emb.shape[1])
    per_type, total = {}, 0.0
    for t in KTYPES:
        t1 = time.perf_counter()
        ref.quantize(t, xe, imx_emb, threads=threads)
        dt_t = time.perf_counter() - t1
        total += dt_t
        per_type[NAMES[t]] = {"GB_s": round(2 * xe.size / dt_t / 1e9, 4), "sample": f"token_embd rows 0..{rows}, imatrix"}
    # configuration 1 (no imatrix) and configuration 3 (imatrix), each type on its own bounded sample
    w1, _ = synth.tensor(1, 0)
    x1 = synth.bf16_to_f32(w1).reshape(w1.shape)
    w3, imx3 = synth.tensor(3, 0)
    x3 = synth.bf16_to_f32(w3).reshape(w3.shape)
    for t, xs, imx, what in [(8, x1, None, "cfg1 3072x1024"), (2, x1, None, "cfg1 3072x1024")] + \
                            [(t, x3, imx3, "cfg3 4096x12288, imatrix") for t in synth.TYPES[3]]:
        r, dt_t = _timed_sample(lambda xx: ref.quantize(t, xx, imx, threads=threads), xs, type_s)
        per_type[NAMES[t]] = {"GB_s": round(2 * r * xs.shape[1] / dt_t / 1e9, 4), "sample": f"{what}: rows 0..{r}"}
    # QR encode of configuration 1 (Q8_0 / Q4_0 prediction, 1% of the blocks perturbed): the oracle's port
    qr_cpu = {}
    sd = w1.reshape(-1).view(np.uint8).tobytes()
    for t, bs in ((8, 34), (2, 18)):
        P = ref.quantize(t, x1, None, threads=threads)
        g = np.random.Generator(np.random.PCG64(1234 + t))
        Fb = P.copy().reshape(-1, bs)
        idx = g.choice(len(Fb), size=len(Fb) // 100, replace=False)
        Fb[idx, g.integers(0, bs, len(idx))] ^= np.uint8(0x10)
        t1 = time.perf_counter()
        oqr.encode(t, Fb.tobytes(), P.tobytes(), sd, 30, w1.shape[1])
        dt_t = time.perf_counter() - t1
        qr_cpu[NAMES[t]] = {"encode_GB_s_bf16": round(2 * w1.size / dt_t / 1e9, 4), "encode_s": round(dt_t, 3)}
    return {"value": round(5 * 2 * xe.size / total / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "reference",
            "sample": f"token_embd rows 0..{rows} ({xe.size} weights) x Q2_K..Q6_K with imatrix, "
                      f"oracle/_ref built from the reference's ggml-quants.c, {threads} threads, {total:.1f} s",
            "cpu_model": _cpu_model(), "per_type": per_type,
            "per_type_note": f"GB/s of BF16 in, oracle/_ref (the reference's own C quantizers), {threads} threads, rows "
                             "split into contiguous parts as the reference's CPU entry does (requant.py:115-134)",
            "qr_cfg1": qr_cpu, "qr_cfg1_note": "QR encode of the whole configuration-1 tensor by oracle/qr.py, the "
                                                "oracle's numpy restatement (kind: port), one core"}


def _profiled_traffic(kernel):
    """HBM bytes per launch of a kernel on the embedding, from the rocprofv3 FETCH_SIZE/WRITE_SIZE
    passes summarised in profiles/ (scaled by the copy-kernel factors recorded there)"""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    return json.load(open(p))["bytes_per_launch"].get(kernel)


SIMDS, CLOCK_GHZ = 1024, 2.4
PROBE_BLOCKS, PROBE_ITERS = 4096, 4000
PROBES = ((0, "v_fma_f32"), (1, "v_add_f32"), (2, "v_xor_b32+v_add_u32"), (3, "v_fma_f32 with v_xor_b32+v_add_u32"),
          (4, "v_mul_f32 with v_add_f32"), (5, "v_mul_f32"))


def valu_probe(stream, reps=5):
    """the VALU yardstick (spa_valu_probe): loops of known length of plain 32-bit VALU instructions,
    timed with HIP events on the bench stream -> instruction rate, lane-ops/s and cycles per
    instruction per SIMD at the 2.4 GHz peak clock. None of them dual-issues (SQ_ACTIVE_INST_VALU2 = 0
    in the counter pass): the fastest is the single-issue rate, one wave64 instruction per SIMD per
    quad-cycle; two per quad-cycle is the issue limit (profiles/valu.json)."""
    from seedpack_amd import device as dev
    from seedpack_amd._lib import check, lib
    out = dev.DeviceArray(PROBE_BLOCKS * 256, np.float32)
    res = {"workgroups": PROBE_BLOCKS, "loop_trips": PROBE_ITERS}
    for op, name in PROBES:
        insts = int(lib().spa_valu_probe_insts(op, PROBE_BLOCKS, PROBE_ITERS))
        check(lib().spa_valu_probe(op, PROBE_BLOCKS, PROBE_ITERS, out.ptr, stream.handle))
        best = None
        for _ in range(reps):
            e0, e1 = dev.Event(), dev.Event()
            e0.record(stream.handle)
            check(lib().spa_valu_probe(op, PROBE_BLOCKS, PROBE_ITERS, out.ptr, stream.handle))
            e1.record(stream.handle)
            stream.synchronize()
            ms = e0.elapsed_ms(e1)
            best = ms if best is None else min(best, ms)
        rate = insts / (best / 1e3)
        res[name] = {"ms": round(best, 4), "wave64_valu_insts": insts, "T_lane_ops_s": round(rate * 64 / 1e12, 2),
                     "cycles_per_inst_per_simd_at_2p4GHz": round(SIMDS * CLOCK_GHZ * 1e9 / rate, 3)}
        log(f"bench: VALU probe {name}: {best:.3f} ms, {rate * 64 / 1e12:.1f} T lane-ops/s")
    res["single_issue_T_lane_ops_s"] = max(v["T_lane_ops_s"] for v in res.values() if isinstance(v, dict))
    res["dual_issue_peak_T_lane_ops_s"] = round(2 * res["single_issue_T_lane_ops_s"], 2)
    return res


def _profiled_valu(kernel):
    """VALU lane-ops per launch of a kernel on the embedding: SQ_INSTS_VALU x 64 from the rocprofv3
    counter pass summarised in profiles/"""
    p = os.path.join(ROOT, "profiles", "valu.json")
    if not os.path.exists(p):
        return None
    d = json.load(open(p))
    n = d["insts_valu_per_launch"].get(kernel)
    return None if n is None else n * d["lane_ops_per_instruction"]


def _profiled_issue(kernel):
    """share of the SIMDs' quad-cycles issuing at least one VALU instruction, from the counter pass"""
    p = os.path.join(ROOT, "profiles", "valu.json")
    if not os.path.exists(p):
        return None
    return json.load(open(p)).get("issue", {}).get(kernel, {}).get("issue_slot_occupancy")


def _cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def profile_pass():
    """each kernel of the step once, after one warm-up launch, plus the copy yardstick"""
    from seedpack_amd import device as dev
    from seedpack_amd import synth
    from seedpack_amd._lib import check, lib
    from seedpack_amd.gpuquant import quantize_into
    from seedpack_amd.requant import NAMES, row_size

    w, imx = synth.tensor(2, 0)
    src = dev.DeviceArray.from_host(w.reshape(-1))
    dimx = dev.DeviceArray.from_host(imx)
    for t in [8, 2] + KTYPES:
        out = dev.DeviceArray(w.shape[0] * row_size(t, w.shape[1]), np.uint8)
        m = None if t in (8, 2) else dimx
        for _ in range(2):
            quantize_into(t, src, w.shape[1], out, m)
        dev.synchronize()
        log(f"profile: {NAMES[t]} token_embd {w.shape[0]}x{w.shape[1]} x2 launches, "
            f"algorithmic bytes/launch {alg_bytes(t, w.size, w.shape[1], m is not None)}")
    w3, imx3 = synth.tensor(3, 0)
    src3 = dev.DeviceArray.from_host(w3.reshape(-1))
    dimx3 = dev.DeviceArray.from_host(imx3)
    for t in synth.TYPES[3]:
        out = dev.DeviceArray(w3.shape[0] * row_size(t, w3.shape[1]), np.uint8)
        for _ in range(2):
            quantize_into(t, src3, w3.shape[1], out, dimx3)
        dev.synchronize()
        log(f"profile: {NAMES[t]} cfg3 {w3.shape[0]}x{w3.shape[1]} x2 launches, "
            f"algorithmic bytes/launch {alg_bytes(t, w3.size, w3.shape[1], True)}")
        del out
    nb = 512 << 20
    a, b = dev.DeviceArray(nb, np.uint8), dev.DeviceArray(nb, np.uint8)
    for _ in range(2):
        check(lib().spa_copy(b.ptr, a.ptr, nb, None))
    dev.synchronize()
    log(f"profile: k_copy16 {nb} bytes x2 launches (reads {nb}, writes {nb})")
    pr = dev.DeviceArray(PROBE_BLOCKS * 256, np.float32)
    for op, name in PROBES:
        for _ in range(2):
            check(lib().spa_valu_probe(op, PROBE_BLOCKS, PROBE_ITERS, pr.ptr, None))
        dev.synchronize()
        log(f"profile: k_valu_probe<{op}> ({name}) x2 launches, "
            f"{lib().spa_valu_probe_insts(op, PROBE_BLOCKS, PROBE_ITERS)} loop VALU instructions per launch")


def iquant_cfg3(stream, reps=2, types=None):
    """configuration 3: the i-quants (or `types`) with the imatrix on the 4096x12288 and 12288x4096
    Student-t tensors, each type launched once untimed, then `reps` times between HIP events on the
    bench stream"""
    from seedpack_amd import device as dev
    from seedpack_amd import synth
    from seedpack_amd.gpuquant import quantize_into
    from seedpack_amd.requant import NAMES, row_size
    res = {}
    for ti in (0, 1):
        w, imx = synth.tensor(3, ti)
        src = dev.DeviceArray.from_host(w.reshape(-1), stream.handle)
        dimx = dev.DeviceArray.from_host(imx, stream.handle)
        for t in types or synth.TYPES[3]:
            out = dev.DeviceArray(w.shape[0] * row_size(t, w.shape[1]), np.uint8)
            quantize_into(t, src, w.shape[1], out, dimx, 0, stream.handle)
            e0, e1 = dev.Event(), dev.Event()
            e0.record(stream.handle)
            for _ in range(reps):
                quantize_into(t, src, w.shape[1], out, dimx, 0, stream.handle)
            e1.record(stream.handle)
            ms = e0.elapsed_ms(e1) / reps
            key = NAMES[t]
            ent = res.setdefault(key, {"ms": 0.0, "bf16_bytes": 0})
            ent["ms"] += ms
            ent["bf16_bytes"] += 2 * w.size
            log(f"bench: cfg3 {NAMES[t]} t{ti} {w.shape[0]}x{w.shape[1]}: {ms:.3f} ms/launch")
            del out
        del src, dimx
    for k, e in res.items():
        e["GB_s"] = round(e["bf16_bytes"] / (e["ms"] / 1e3) / 1e9, 2)
        e["ms"] = round(e["ms"], 3)
    return res


def qr_cfg3(stream, reps=2):
    """grid-type residual coding on the configuration-3 4096x12288 tensor: prediction = the HIP
    quantizer's bytes (imatrix), file = 1% of its blocks perturbed (one byte each); QR encode and
    decode wall time per call with inputs resident on the device"""
    from seedpack_amd import device as dev
    from seedpack_amd import qr, synth
    from seedpack_amd.gpuquant import quantize_into
    from seedpack_amd.requant import NAMES, row_size
    w, imx = synth.tensor(3, 0)
    sd = dev.DeviceArray.from_host(w.reshape(-1).view(np.uint8), stream.handle)
    dimx = dev.DeviceArray.from_host(imx, stream.handle)
    res = {}
    for t in [17, 16, 18, 19, 29]:
        P = dev.DeviceArray(w.shape[0] * row_size(t, w.shape[1]), np.uint8)
        quantize_into(t, sd.view(0, (w.size,), np.uint16), w.shape[1], P, dimx, 0, stream.handle)
        Ph = P.to_host(stream=stream.handle)
        g = np.random.Generator(np.random.PCG64(77 + t))
        Fb = Ph.copy().reshape(-1, qr.BS[t])
        idx = g.choice(len(Fb), size=len(Fb) // 100, replace=False)
        Fb[idx, g.integers(0, qr.BS[t], len(idx))] ^= np.uint8(0x21)
        F = dev.DeviceArray.from_host(Fb.reshape(-1), stream.handle)
        item = [(F, P, 0, 30, w.shape[1], 0)]
        parts = qr.encode_parts(t, item, sd, dimx, stream=stream.handle)
        t0 = time.perf_counter()
        for _ in range(reps):
            parts = qr.encode_parts(t, item, sd, dimx, stream=stream.handle)
        enc = (time.perf_counter() - t0) / reps
        args = (parts["freq"], parts["used"], parts["lens"], parts["stream"].tobytes(), [(P, 0, 30, w.shape[1], 0)], sd, dimx)
        back = qr.decode_parts(t, *args, stream=stream.handle)
        stream.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            back = qr.decode_parts(t, *args, stream=stream.handle)
        stream.synchronize()
        dec = (time.perf_counter() - t0) / reps
        ok = back.to_host(stream=stream.handle)[:F.nbytes].tobytes() == Fb.tobytes()
        res[NAMES[t]] = {"file_bytes": int(F.nbytes), "blocks_differing": int(len(idx)), "coded_bytes": int(len(parts["stream"])),
                         "encode_ms": round(enc * 1e3, 3), "decode_ms": round(dec * 1e3, 3),
                         "encode_GB_s_bf16": round(2 * w.size / enc / 1e9, 2),
                         "decode_GB_s_bf16": round(2 * w.size / dec / 1e9, 2), "round_trip_ok": ok}
        log(f"bench: qr cfg3 {NAMES[t]}: {res[NAMES[t]]}")
    return res


def r2_layer(stream):
    """R2 BF16 base codec on a Qwen-9B-shaped block's attn_q (4096x4096) and ffn_down (12288x4096)
    BF16 weights (134 MB, N(0, 0.02)), as configuration 4 applies it to the base: compress (statistics,
    duplicate check, histogram, tables, coding, gather) and decompress, wall time per call"""
    from seedpack_amd import r2, synth
    g = np.random.Generator(np.random.PCG64(0x5EED0040))
    wq = synth.normal_bf16(g, (4096, 4096), 0.02)
    wd = synth.normal_bf16(g, (4096, 12288), 0.02)
    hdr = b"\0" * 4096
    data = hdr + wq.tobytes() + wd.tobytes()
    layout = r2.layout_of([("blk.0.attn_q.weight", 4096, wq.nbytes, 4096),
                           ("blk.0.ffn_down.weight", 4096 + wq.nbytes, wd.nbytes, 12288)], len(data))
    codec = r2.BF16v2(stream=stream.handle)
    parts = codec.compress(data, layout)
    t0 = time.perf_counter()
    parts = codec.compress(data, layout)
    enc = time.perf_counter() - t0
    out = codec.decompress(parts)
    t0 = time.perf_counter()
    out = codec.decompress(parts)
    dec = time.perf_counter() - t0
    nb = wq.nbytes + wd.nbytes
    ok = out[4096:].tobytes() == data[4096:]
    res = {"bf16_bytes": nb, "coded_bytes": len(parts["stream"]), "ratio": round(len(parts["stream"]) / nb, 4),
           "compress_s": round(enc, 3), "decompress_s": round(dec, 3), "compress_GB_s": round(nb / enc / 1e9, 3),
           "decompress_GB_s": round(nb / dec / 1e9, 3), "round_trip_ok": ok,
           "note": "host<->device copies included (the file is read from and written to host memory)"}
    log(f"bench: r2 {res}")
    return res


def cfg4_matrices(layers=36):
    """configuration 4's 2-D BF16 matrices (name, rows, row length): 36 Qwen3.5-9B-shaped blocks and
    the 151936-row embedding and output, 8,190,427,136 weights"""
    from seedpack_amd import synth
    return [(n, s[1], s[0]) for n, s, t in synth.qwen_tensors(layers, norms=False)]


def cfg4_base(stream, layers=36):
    """configuration 4's BF16 file region in HBM: every 2-D matrix back to back (32-byte aligned after
    a 4 KB header), N(0, 0.02) from a counter-based generator per tensor -> (array, [(name, offset,
    bytes, row length)], file size)"""
    from seedpack_amd import device as dev
    from seedpack_amd._lib import check, lib
    pos, ts = 4096, []
    for name, rows, rl in cfg4_matrices(layers):
        pos += (-pos) % 32
        ts.append((name, pos, rows * rl * 2, rl))
        pos += rows * rl * 2
    d = dev.DeviceArray(pos, np.uint8).zero(stream.handle)
    for k, (name, off, nb, rl) in enumerate(ts):
        check(lib().spa_synth_normal_bf16(d.ptr + off, nb // 2, 0x5EED0040 + k, 0.02, stream.handle))
    stream.synchronize()
    return d, ts, pos


# configuration 4's quant files: the 20 quantizers, and a Q4_K_M-like mix (Q6_K for attn_v, ffn_down
# and output, Q4_K elsewhere)
PACK_TYPES = [2, 3, 6, 7, 8, 42, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29]


class HbmPeak:
    """peak device memory in use (hipMemGetInfo polled every 20 ms on a thread) between start() and stop()"""

    def __init__(self):
        from seedpack_amd import device as dev
        self.dev, self.peak, self.run = dev, 0, False

    def _poll(self):
        while self.run:
            free, total = self.dev.mem_info()
            self.peak = max(self.peak, total - free)
            time.sleep(0.02)

    def start(self):
        free, total = self.dev.mem_info()
        self.base, self.peak, self.run = total - free, total - free, True
        self.t = threading.Thread(target=self._poll, daemon=True)
        self.t.start()
        return self

    def stop(self):
        self.run = False
        self.t.join()
        return self.peak


def repo_cfg45(layers=36, files=None, root="/dev/shm/spa_bench_repo", keep=False, reuse=False, write_only=False,
               bases_in_hbm=None, blocking_waits=True):
    """configurations 4 and 5 from host files, as the reference's CLI measures them (cli.py:288-292,
    :441): a synthetic Qwen3.5-9B-shaped repository (BF16 GGUF with a 151,936-token BPE tokenizer,
    imatrix.dat, README.md, 21 quantized GGUFs made by this library's quantizers with 1% of their
    blocks changed) written to host files (untimed); then, timed, seedpack_amd.repo's pack of the
    directory into a .seedpack archive (file reads, the catalog's BLAKE3 of every file (on the device),
    regrowth / comparison / QR coding on the device, the R2 base codec, zstd of the residuals, the
    container), and the extract of the Q4_K_M-like and IQ2_XS files from that archive (residual zstd,
    regrowth, QR decode, BLAKE3 check, files written). Peak HBM by hipMemGetInfo polling. The extracted files are
    compared byte for byte with the originals. reuse: the repository a previous write_only call left
    in root is packed (a kernel-trace run then sees the pack and the extract only). bases_in_hbm False:
    the base kept in host memory by the pack and decoded window by window by the extract, which then
    writes the base file too."""
    import shutil
    from seedpack_amd import device as dev
    from seedpack_amd import repo, synth
    from seedpack_amd.requant import NAMES
    qf = {f"model-{NAMES[t]}.gguf": (lambda name, t=t: t) for t in PACK_TYPES}
    qf["model-Q4_K_M.gguf"] = synth.q4_k_m
    if files is not None:
        qf = {k: v for k, v in qf.items() if k in files}
    src, arc_dir, out = os.path.join(root, "repo"), os.path.join(root, "arc"), os.path.join(root, "out")
    done = os.path.join(root, "written.json")
    reuse = reuse and os.path.exists(done)
    keep = keep or reuse
    for d in ((arc_dir, out) if reuse else (src, arc_dir, out)):
        shutil.rmtree(d, ignore_errors=True)
        os.makedirs(d)
    try:
        if reuse:
            sizes = json.load(open(done))
            log(f"bench: repo reused: {len(sizes)} files, {sum(sizes.values()) / 1e9:.1f} GB")
        else:
            t0 = time.perf_counter()
            s = dev.Stream()
            sizes = synth.write_repo(src, synth.qwen_tensors(layers), qf, per_million=10000, nmerge=151936 - 256 - 8,
                                     stream=s, log=log)
            dev.synchronize()
            json.dump(sizes, open(done, "w"))
            log(f"bench: repo written: {len(sizes)} files, {sum(sizes.values()) / 1e9:.1f} GB in {time.perf_counter() - t0:.1f} s")
        if write_only:
            keep = True
            return None, None
        arc = os.path.join(arc_dir, "model.seedpack")
        # (untimed) the device blocks that earlier sections left cached are released, so that the pack
        # starts as it does in a process of its own
        dev.release_cached()
        peak = HbmPeak().start()
        st = repo.Packer(verbose=True, bases_in_hbm=bases_in_hbm, blocking_waits=blocking_waits).pack([src], arc)
        pk_peak = peak.stop()
        log(f"bench: pack {st['input_bytes'] / 1e9:.1f} GB -> {st['archive_bytes'] / 1e9:.2f} GB in {st['seconds']:.1f} s "
            f"= {st['GB_s']:.2f} GB/s, peak HBM {pk_peak / 1e9:.1f} GB (residuals waiting in HBM: at most "
            f"{st['residuals_in_hbm_peak'] / 1e9:.1f} GB)")
        for f in st["files"]:
            log(f"bench:   {f}")
        log(f"bench: pack cpu {st['cpu']}")
        log(f"bench: pack started at {st['clock_start_s']:.6f} s (perf_counter)")
        want = [n for n in ("model-Q4_K_M.gguf", "model-IQ2_XS.gguf") if n in qf]
        if bases_in_hbm is False:
            want.append("model-BF16.gguf")
        dev.release_cached()
        peak = HbmPeak().start()
        ex = repo.Unpacker(verbose=True, bases_in_hbm=bases_in_hbm, blocking_waits=blocking_waits).run(arc, out, want)
        up_peak = peak.stop()
        same = all(_same_file(os.path.join(src, n), os.path.join(out, n)) for n in want)
        log(f"bench: extract {ex['bytes'] / 1e9:.2f} GB in {ex['seconds']:.2f} s = {ex['GB_s']:.2f} GB/s, "
            f"byte-identical {same}")
        pack = {"workload": f"cfg4: {len(sizes)} files from host files ({layers} blocks, 21 quant files, 1% of each "
                            "file's blocks changed) -> .seedpack", "input_bytes": st["input_bytes"],
                "archive_bytes": st["archive_bytes"], "ratio": round(st["archive_bytes"] / st["input_bytes"], 4),
                "pack_s": round(st["seconds"], 2), "pack_GB_s": round(st["GB_s"], 3), "peak_hbm_GB": round(pk_peak / 1e9, 1),
                "stats": st["stats"], "phases_s": st.get("phases"), "host_cpu_s": st.get("cpu")}
        unpack = {"workload": "cfg5: Q4_K_M-like and IQ2_XS extracted from the cfg4 archive (files written, catalog checksums checked)"
                              + (", and the BF16 base decoded window by window" if bases_in_hbm is False else ""),
                  "written_bytes": ex["bytes"], "extract_s": round(ex["seconds"], 2), "GB_s_written": round(ex["GB_s"], 3),
                  "checksums_ok": not ex["bad"] and not ex["missing"], "byte_identical": same,
                  "peak_hbm_GB": round(up_peak / 1e9, 1)}
        return pack, unpack
    finally:
        if not keep:
            shutil.rmtree(root, ignore_errors=True)


def _same_file(a, b, chunk=1 << 28):
    with open(a, "rb") as fa, open(b, "rb") as fb:
        while True:
            x, y = fa.read(chunk), fb.read(chunk)
            if x != y:
                return False
            if not x:
                return True


def r2_cfg4(stream, layers=36):
    """R2 BF16 base codec on configuration 4's whole base (every 2-D matrix, 16.4 GB), generated in
    HBM (N(0, 0.02), a counter-based generator per tensor): compress of the resident file and
    decompress back into HBM, wall time per call (the coded stream is read back to / sent from host
    memory, the contract of the reference's compress_parts / decompress), plus the device phases
    timed with HIP events on the stream; round trip checked on the device"""
    from seedpack_amd import device as dev
    from seedpack_amd import framing, r2, residual
    from seedpack_amd._lib import check, lib
    d, ts, pos = cfg4_base(stream, layers)
    layout = r2.layout_of(ts, pos)
    nb_all = sum(t[2] for t in ts)
    codec = r2.BF16v2(stream=stream.handle, timing=True)
    warm = r2.layout_of(ts[1:8], ts[7][1] + ts[7][2])          # one block: loads the kernels
    codec.decompress(codec.compress(d, warm), device=True)
    t0 = time.perf_counter()
    parts = codec.compress(d, layout)
    enc = time.perf_counter() - t0
    enc_ph = codec.last_timing
    del parts["arrays"]
    t0 = time.perf_counter()
    back = codec.decompress(parts, device=True)
    dec = time.perf_counter() - t0
    dec_ph = codec.last_timing
    bad = sum(residual.diff_count(d.view(off, (nb,), np.uint8), back.view(off, (nb,), np.uint8), stream.handle)
              for _, off, nb, _ in ts)
    coded = framing.nbytes(parts["stream"])
    enc_dev = sum(v for k, v in enc_ph.items() if k != "host_s") / 1e3
    dec_dev = sum(v for k, v in dec_ph.items() if k != "host_s") / 1e3
    res = {"workload": f"cfg4 base: {len(ts)} matrices ({layers} blocks + token_embd + output)", "bf16_bytes": nb_all,
           "segments": nb_all // 2 // r2.SEG, "coded_bytes": coded, "ratio": round(coded / nb_all, 4),
           "compress_s": round(enc, 3), "decompress_s": round(dec, 3),
           "compress_GB_s": round(nb_all / enc / 1e9, 2), "decompress_GB_s": round(nb_all / dec / 1e9, 2),
           "compress_device_ms": {k: round(v, 2) for k, v in enc_ph.items() if k != "host_s"},
           "decompress_device_ms": {k: round(v, 2) for k, v in dec_ph.items() if k != "host_s"},
           "compress_host_s": enc_ph.get("host_s"), "decompress_host_s": dec_ph.get("host_s"),
           "compress_device_GB_s": round(nb_all / enc_dev / 1e9, 2), "decompress_device_GB_s": round(nb_all / dec_dev / 1e9, 2),
           "round_trip_bytes_differing": int(bad),
           "note": "wall includes the per-tensor statistics readback, host table normalisation and the stream's "
                   "host transfers; *_device_* sums the kernel phases"}
    log(f"bench: r2 cfg4 {res}")
    del back, d
    return res


def dequant_cfg2(stream, dsrc, dimx, reps=10):
    """dequantizers (GPUQuant.dequantize) on the configuration-2 embedding quantized to each K-quant
    and Q8_0 / Q4_0: float32 out; HBM-bound (4 bytes written per weight + the block bytes read)"""
    from seedpack_amd import device as dev
    from seedpack_amd._lib import check, lib
    from seedpack_amd.gpuquant import quantize_into
    from seedpack_amd.requant import NAMES, row_size
    rows, npr = 151936, 1024
    out = dev.DeviceArray(rows * npr, np.float32)
    res = {}
    for t in (8, 2) + tuple(KTYPES):
        q = dev.DeviceArray(rows * row_size(t, npr), np.uint8)
        quantize_into(t, dsrc, npr, q, None if t in (8, 2) else dimx, 0, stream.handle)
        check(lib().spa_dequantize(t, q.ptr, rows, npr, out.ptr, stream.handle))
        e0, e1 = dev.Event(), dev.Event()
        e0.record(stream.handle)
        for _ in range(reps):
            check(lib().spa_dequantize(t, q.ptr, rows, npr, out.ptr, stream.handle))
        e1.record(stream.handle)
        ms = e0.elapsed_ms(e1) / reps
        nb = q.nbytes + out.nbytes
        res[NAMES[t]] = {"ms": round(ms, 4), "GB_s_f32_out": round(out.nbytes / ms / 1e6, 1),
                         "hbm_frac": round(nb / ms / 1e6 / PEAK_HBM_GBS, 4)}
        del q
    log(f"bench: dequant token_embd {res}")
    return res


def qr_cfg1(stream, reps=3):
    """configuration 1 residual coding: Q8_0 / Q4_0 of the 3072x1024 tensor as the prediction, the file
    is that with 1% of its blocks perturbed (one byte each); QR encode (histogram, tables, coding, gather)
    and decode, inputs resident on the device, wall time per call including the host table step"""
    from seedpack_amd import device as dev
    from seedpack_amd import qr, synth
    from seedpack_amd.gpuquant import quantize_into
    from seedpack_amd.requant import NAMES, row_size
    w, _ = synth.tensor(1, 0)
    sd = dev.DeviceArray.from_host(w.reshape(-1).view(np.uint8), stream.handle)
    src = dev.DeviceArray.from_host(w.reshape(-1), stream.handle)
    res = {}
    for t in (8, 2):
        P = dev.DeviceArray(w.shape[0] * row_size(t, w.shape[1]), np.uint8)
        quantize_into(t, src, w.shape[1], P, None, 0, stream.handle)
        Ph = P.to_host(stream=stream.handle)
        g = np.random.Generator(np.random.PCG64(1234 + t))
        Fb = Ph.copy().reshape(-1, qr.BS[t])
        idx = g.choice(len(Fb), size=len(Fb) // 100, replace=False)
        Fb[idx, g.integers(0, qr.BS[t], len(idx))] ^= np.uint8(0x10)
        F = dev.DeviceArray.from_host(Fb.reshape(-1), stream.handle)
        item = [(F, P, 0, 30, w.shape[1], -1)]
        parts = qr.encode_parts(t, item, sd, stream=stream.handle)
        t0 = time.perf_counter()
        for _ in range(reps):
            parts = qr.encode_parts(t, item, sd, stream=stream.handle)
        enc = (time.perf_counter() - t0) / reps
        args = (parts["freq"], parts["used"], parts["lens"], parts["stream"].tobytes(), [(P, 0, 30, w.shape[1], -1)], sd)
        back = qr.decode_parts(t, *args, stream=stream.handle)
        stream.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            back = qr.decode_parts(t, *args, stream=stream.handle)
        stream.synchronize()
        dec = (time.perf_counter() - t0) / reps
        ok = back.to_host(stream=stream.handle)[:F.nbytes].tobytes() == Fb.tobytes()
        res[NAMES[t]] = {"file_bytes": int(F.nbytes), "coded_bytes": int(len(parts["stream"])),
                         "encode_ms": round(enc * 1e3, 3), "decode_ms": round(dec * 1e3, 3),
                         "encode_GB_s_bf16": round(2 * w.size / enc / 1e9, 2),
                         "decode_GB_s_bf16": round(2 * w.size / dec / 1e9, 2), "round_trip_ok": ok}
        log(f"bench: qr cfg1 {NAMES[t]}: {res[NAMES[t]]}")
    return res


def q8_codec(stream, layers=4):
    """the Q8_0 codec (q8.Q8Parts over M22: a seed's Q8_0 part) on a Qwen3.5-9B-shaped Q8_0 file:
    token_embd and output 151936 x 4096 and `layers` transformer blocks, Q8_0 of N(0, 0.02) weights;
    compress (row planner on token_embd) and decompress timed from a host file to a host file, the
    result byte-identical; per-phase times with the stream drained between phases"""
    from seedpack_amd import device as dev
    from seedpack_amd import gguf, q8
    from seedpack_amd._lib import check, lib
    from seedpack_amd.gpuquant import quantize_into
    st = stream.handle
    shapes = [("token_embd.weight", (4096, 151936))]
    for i in range(layers):
        shapes += [(f"blk.{i}.attn_q.weight", (4096, 4096)), (f"blk.{i}.attn_k.weight", (4096, 1024)),
                   (f"blk.{i}.attn_v.weight", (4096, 1024)), (f"blk.{i}.attn_output.weight", (4096, 4096)),
                   (f"blk.{i}.ffn_gate.weight", (4096, 12288)), (f"blk.{i}.ffn_up.weight", (4096, 12288)),
                   (f"blk.{i}.ffn_down.weight", (12288, 4096))]
    shapes.append(("output.weight", (4096, 151936)))
    head, where, size = gguf.header_bytes({"general.architecture": "qwen35", "general.alignment": 32},
                                          [(n, sh, 8) for n, sh in shapes])
    log(f"bench q8: building a {size / 1e9:.2f} GB Q8_0 file")
    host = dev.pinned(size)
    host[:] = 0
    host[:len(head)] = np.frombuffer(head, np.uint8)
    for k, ((n, sh), (off, nb)) in enumerate(zip(shapes, where)):
        nw = sh[0] * sh[1]
        w = dev.DeviceArray(nw, np.uint16)
        check(lib().spa_synth_normal_bf16(w.ptr, nw, 0x0880 + 7 * k, 0.02, st))
        y = dev.DeviceArray(nb, np.uint8)
        quantize_into(8, w, sh[0], y, None, 0, st)
        check(lib().spa_memcpy_d2h(host[off:].ctypes.data, y.ptr, nb, st))
        del w, y
    stream.synchronize()
    g = gguf.GGUF(host)
    parts = q8.Q8Parts(stream=st, timing=True)
    t0 = time.perf_counter()
    buf = parts.compress(host, g=g)
    t1 = time.perf_counter()
    dec = q8.Q8Parts(stream=st, timing=True)
    out = dec.decompress(buf)
    t2 = time.perf_counter()
    ok = bool(np.array_equal(out, host))
    res = {"file_bytes": size, "coded_bytes": len(buf), "ratio": round(len(buf) / size, 4), "parts": parts.parts,
           "compress_s": round(t1 - t0, 3), "compress_GB_s": round(size / (t1 - t0) / 1e9, 3),
           "decompress_s": round(t2 - t1, 3), "decompress_GB_s": round(size / (t2 - t1) / 1e9, 3),
           "identical": ok, "compress_phases_s": parts.c.timing, "decompress_phases_s": dec.c.timing}
    log(f"bench q8: {res}")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-pass", action="store_true",
                    help="two launches of each kernel (K-quants and Q8_0/Q4_0 on token_embd, the configuration-3 "
                         "i-quants on its 4096x12288 tensor) plus a 512 MiB copy, "
                         "for rocprofv3 counter runs; prints the launch list, no JSON line")
    ap.add_argument("--pack", action="store_true",
                    help="only configurations 4 and 5 (repository pack from host files, extract of two files); prints "
                         "their result, no JSON line")
    ap.add_argument("--pack-layers", type=int, default=36, help="transformer blocks of the --pack model")
    ap.add_argument("--unpack", action="store_true", help="the same as --pack")
    ap.add_argument("--no-repo", action="store_true", help="leave configurations 4 and 5 out of the JSON line")
    ap.add_argument("--pack-files", default=None, help="comma-separated quant files of --pack (default: all 21)")
    ap.add_argument("--repo-dir", default="/dev/shm/spa_bench_repo", help="where --pack writes its repository")
    ap.add_argument("--write-repo", action="store_true",
                    help="only write the --pack repository into --repo-dir and keep it (for a later --reuse-repo run)")
    ap.add_argument("--reuse-repo", action="store_true",
                    help="--pack on the repository a --write-repo run left in --repo-dir (kept)")
    ap.add_argument("--bases-host", action="store_true",
                    help="--pack with the BF16 base kept in host memory (pack) and decoded window by window from the "
                         "archive (extract, which writes the base file too), as for a base bigger than HBM")
    ap.add_argument("--spin-waits", action="store_true",
                    help="--pack with the library's waits for the device spinning (the runtime's stream "
                         "synchronisation) instead of blocking on an event")
    ap.add_argument("--q8", action="store_true",
                    help="only the Q8_0 codec (a seed's Q8_0 part) on a Qwen3.5-9B-shaped Q8_0 file; prints its "
                         "result, no JSON line")
    ap.add_argument("--q8-layers", type=int, default=4, help="transformer blocks of the --q8 file")
    ap.add_argument("--codecs", action="store_true",
                    help="only the coding stages (QR on configurations 1 and 3, the R2 base codec), for rocprofv3 "
                         "kernel-trace runs; prints their results, no JSON line")
    a = ap.parse_args()
    if a.profile_pass:
        return profile_pass()
    if a.pack or a.unpack or a.write_repo:
        files = a.pack_files.split(",") if a.pack_files else None
        pk, upk = repo_cfg45(layers=a.pack_layers, files=files, root=a.repo_dir, reuse=a.reuse_repo,
                             write_only=a.write_repo, bases_in_hbm=False if a.bases_host else None,
                             blocking_waits=not a.spin_waits)
        if not a.write_repo:
            print(json.dumps({"pack_cfg4": pk, "unpack_cfg5": upk}))
        return None
    if a.q8:
        from seedpack_amd import device as dev
        print(json.dumps({"q8_codec": q8_codec(dev.Stream(), a.q8_layers)}))
        return None
    if a.codecs:
        from seedpack_amd import device as dev
        stream = dev.Stream()
        qr_cfg1(stream)
        qr_cfg3(stream)
        r2_layer(stream)
        r2_cfg4(stream)
        return None
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {a.gpus} requested); the path shards by rows "
              "with no exchange, so N GPUs is N independent copies of this run", file=sys.stderr)
        sys.exit(2)

    from seedpack_amd import device as dev
    from seedpack_amd import synth
    from seedpack_amd.gpuquant import quantize_into
    from seedpack_amd.requant import NAMES, row_size

    log("bench: generating synthetic inputs")
    tensors = {"token_embd": synth.tensor(2, 0), "ffn_down": synth.tensor(2, 1)}
    stream = dev.Stream()
    dsrc, dimx, dout = {}, {}, {}
    for name, (w, imx) in tensors.items():
        dsrc[name] = dev.DeviceArray.from_host(w.reshape(-1), stream.handle)
        dimx[name] = dev.DeviceArray.from_host(imx, stream.handle)
        for t in KTYPES:
            dout[(name, t)] = dev.DeviceArray(w.shape[0] * row_size(t, w.shape[1]), np.uint8)
    launches = [(t, name) for t in KTYPES for name in tensors]
    ev = {k: (dev.Event(), dev.Event()) for k in launches}

    def step(record):
        for (t, name) in launches:
            w = tensors[name][0]
            if record:
                ev[(t, name)][0].record(stream.handle)
            quantize_into(t, dsrc[name], w.shape[1], dout[(name, t)], dimx[name], 0, stream.handle)
            if record:
                ev[(t, name)][1].record(stream.handle)

    log("bench: warmup")
    for _ in range(a.warmup):
        step(False)
    stream.synchronize()
    dev.synchronize()
    per = {k: 0.0 for k in launches}
    log(f"bench: timing {a.steps} steps")
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step(True)
        stream.synchronize()
        for k in launches:
            per[k] += ev[k][0].elapsed_ms(ev[k][1])
    dev.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / a.steps
    bf16_bytes = sum(2 * tensors[n][0].size for (_, n) in launches)
    value = bf16_bytes / (ms_step / 1e3) / 1e9

    per_type = {}
    for t in KTYPES:
        ms = sum(per[(t, n)] for n in tensors) / a.steps
        nb = sum(2 * tensors[n][0].size for n in tensors)
        per_type[NAMES[t]] = {"GB_s": round(nb / (ms / 1e3) / 1e9, 2), "ms": round(ms, 3)}
    dom = max(launches, key=lambda k: per[k])
    t, n = dom
    w = tensors[n][0]
    dom_ms = per[dom] / a.steps
    ab = alg_bytes(t, w.size, w.shape[1], True)
    achieved = ab / (dom_ms / 1e3) / 1e9
    kname = NAMES[t].replace("_", "")
    traffic = _profiled_traffic(kname) if n == "token_embd" else None
    ops = _profiled_valu(kname) if n == "token_embd" else None
    hbm = {"achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 5),
           "algorithmic_bytes": ab}
    kdesc = f"k_kquant<{NAMES[t]}> on {n} {w.shape[0]}x{w.shape[1]}"
    probe = valu_probe(stream)
    if ops:
        # the K-quant searches are VALU-bound: the roof is the VALU issue limit, two wave64 instructions
        # per SIMD per quad-cycle, at the quad-cycle rate the probe measures in this run; HBM beside it
        va = ops / (dom_ms / 1e3) / 1e12
        peak = probe["dual_issue_peak_T_lane_ops_s"]
        roofline = {"bound": "valu", "kernel": kdesc, "achieved": round(va, 2), "peak": peak,
                    "unit": "T lane-ops/s", "frac": round(va / peak, 4), "traffic": traffic,
                    "valu_lane_ops_per_launch": ops, "avg_launch_ms": round(dom_ms, 4), "hbm": hbm,
                    "issue_slot_occupancy": _profiled_issue(kname), "single_issue_peak": probe["single_issue_T_lane_ops_s"],
                    "frac_of_fp32_tflops": round(va / 157.3, 4), "valu_probe": probe,
                    "note": "lane-ops = SQ_INSTS_VALU x 64 per launch (exact: profiles/valu.json) over the live launch time; "
                            "peak = 2 x the single-issue rate the VALU probe measures in this run (spa_valu_probe: "
                            "plain 32-bit loops, no dual issue); issue_slot_occupancy = quad-cycles issuing at least "
                            "one VALU instruction (SQ_ACTIVE_INST_VALU - SQ_ACTIVE_INST_VALU2 over the SIMDs' "
                            "quad-cycles, counter pass); frac_of_fp32_tflops counts a lane-op as one operation "
                            "against the published 157.3 TFLOP/s (packed FP32, FMA = 2)"}
    else:
        roofline = {"bound": "hbm", "kernel": kdesc, **hbm, "traffic": traffic, "avg_launch_ms": round(dom_ms, 4),
                    "note": "no VALU count profiled for this launch: HBM fraction only"}

    # HBM-bound legacy types: configuration 1 tensor and the embedding, Q8_0 / Q4_0 without imatrix
    legacy = {}
    w1, _ = synth.tensor(1, 0)
    d1 = dev.DeviceArray.from_host(w1.reshape(-1), stream.handle)
    for t in (8, 2):
        for name, src, shape in (("cfg1", d1, w1.shape), ("token_embd", dsrc["token_embd"], tensors["token_embd"][0].shape)):
            out = dev.DeviceArray(shape[0] * row_size(t, shape[1]), np.uint8)
            e0, e1 = dev.Event(), dev.Event()
            for _ in range(2):
                quantize_into(t, src, shape[1], out, None, 0, stream.handle)
            reps = 20
            e0.record(stream.handle)
            for _ in range(reps):
                quantize_into(t, src, shape[1], out, None, 0, stream.handle)
            e1.record(stream.handle)
            ms = e0.elapsed_ms(e1) / reps
            nw = shape[0] * shape[1]
            legacy[f"{NAMES[t]}_{name}"] = {"GB_s_bf16_in": round(2 * nw / (ms / 1e3) / 1e9, 1), "ms": round(ms, 4),
                                           "hbm_frac": round(alg_bytes(t, nw, shape[1], False) / (ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4)}

    dqb = dequant_cfg2(stream, dsrc["token_embd"], dimx["token_embd"])
    iq = iquant_cfg3(stream)
    # the imatrix legacy types on the same tensors (row statistics launch + quantizer)
    lq = iquant_cfg3(stream, 5, [2, 3, 6, 7])
    qrb = qr_cfg1(stream)
    qrg = qr_cfg3(stream)
    r2b = r2_layer(stream)
    r2c = r2_cfg4(stream)
    pk, upk = (None, None) if a.no_repo else repo_cfg45()
    cpu = None if a.no_cpu else cpu_baseline(tensors)
    line = {"metric": "requant GB/s (BF16 in), K-quant family Q2_K..Q6_K with imatrix", "value": round(value, 3),
            "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_step, 3),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded N(0,0.02) BF16, LogNormal(0,1) imatrix)",
            "config": {"workload": "cfg2: Q2_K,Q3_K,Q4_K,Q5_K,Q6_K (imatrix) on token_embd 151936x1024 + ffn_down 1024x3072",
                       "bf16_bytes_per_step": bf16_bytes, "launches_per_step": len(launches)},
            "per_type": per_type, "legacy_hbm_types": legacy, "iquant_cfg3": iq, "legacy_imatrix_cfg3": lq, "dequant_token_embd": dqb, "qr_cfg1": qrb, "qr_cfg3": qrg, "r2_base": r2b, "r2_cfg4": r2c,
            "pack_cfg4": pk, "unpack_cfg5": upk,
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
