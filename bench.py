"""Paged GQA decode attention + KV append on one MI355X.

Workload (the HBM-scale decode configuration): 256 lanes, each with a
32768-token TinyLlama-shaped context (22 layers, 4 KV heads x 64 dims fp16,
32 query heads) held in 64-token extent pages whose slot ids are a seeded
permutation of the pool (~189 GB of KV), plus trailing 8-token micro pages
for the appended tokens.  One step = reserve one token per lane, then for
every layer: append the new K/V of every lane (one batched kernel) and fused
split-K GQA decode attention for all lanes (one kernel + merge), then commit.
With --path engine (default) the step goes through the engine API
(reserveToken / writeLayerBatch / attendLayerBatch / commit, contexts built by
bulk prefill + promotion); with --path kernel the bench builds the page tables
itself and calls the C-ABI kernels directly.

Prints one JSON line (see the contract in the repository's docs).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
from _loader import load_package  # noqa: E402

PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


_HOST_CPU = None


def host_cpu() -> dict:
    """The host CPU the baselines run on, as lscpu reports it (model, sockets, cores per socket,
    threads per core, logical CPUs), plus the CPUs this process may use (its affinity) and
    os.cpu_count()."""
    global _HOST_CPU
    if _HOST_CPU is None:
        info = {"model": platform.processor() or platform.machine()}
        try:
            import subprocess
            out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
            fields = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
            fields = {k.strip(): v.strip() for k, v in fields.items()}
            for key, name in (("Model name", "model"), ("Socket(s)", "sockets"),
                              ("Core(s) per socket", "cores_per_socket"), ("Thread(s) per core", "threads_per_core"),
                              ("CPU(s)", "logical_cpus")):
                if key in fields:
                    info[name] = int(fields[key]) if fields[key].isdigit() else fields[key]
        except (OSError, ValueError, subprocess.SubprocessError):
            pass
        try:
            info["usable_cpus"] = len(os.sched_getaffinity(0))
        except (AttributeError, OSError):
            pass
        info["os_cpu_count"] = os.cpu_count()
        _HOST_CPU = info
    return _HOST_CPU


def cpu_on_host(cpu: dict | None) -> dict | None:
    """A cpu_baseline object with the host CPU it was measured on (None when the baseline was
    skipped)."""
    if cpu is None:
        return None
    cpu["host"] = host_cpu()
    return cpu


def permutation(seed: int, n: int) -> np.ndarray:
    """splitmix64 Fisher-Yates (kimkv_seeded_permutation), vectorised over the draws."""
    mask = np.uint64(0xFFFFFFFFFFFFFFFF)
    steps = np.arange(1, n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (np.uint64(seed) + steps * np.uint64(0x9E3779B97F4A7C15)) & mask
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    out = np.arange(n, dtype=np.uint32)
    bounds = np.arange(n, 1, -1, dtype=np.uint64)
    js = (z % bounds).astype(np.int64)
    for k, i in enumerate(range(n, 1, -1)):
        j = js[k]
        out[i - 1], out[j] = out[j], out[i - 1]
    return out


class Workload:
    def __init__(self, dev, lanes, context, layers, kv_heads, head_dim, query_heads, total_steps, seed,
                 permute=True):
        self.dev = dev
        self.lanes, self.context, self.L = lanes, context, layers
        self.H, self.D, self.QH = kv_heads, head_dim, query_heads
        self.total_steps = total_steps
        self.seed = seed
        self.decode_mode = "plan"
        self.ext_per_lane = context // 64
        assert context % 64 == 0
        self.micro_per_lane = (total_steps + 7) // 8
        self.max_entries = self.ext_per_lane + self.micro_per_lane
        n_ext = lanes * self.ext_per_lane
        n_micro = lanes * self.micro_per_lane + 8
        t0 = time.time()
        self.storage = dev.Storage(layers, kv_heads, head_dim, n_micro, n_ext)
        info = self.storage.info()
        log(f"pools: extent {info.extent_reserved_bytes / 1e9:.1f} GB, micro {info.micro_reserved_bytes / 1e9:.2f} GB "
            f"({time.time() - t0:.1f}s)")
        if permute:
            ext_perm = permutation(seed, n_ext)
            micro_perm = permutation(seed + 1, n_micro)
        else:
            ext_perm = np.arange(n_ext, dtype=np.uint32)
            micro_perm = np.arange(n_micro, dtype=np.uint32)
        # Descriptor arena: lanes x max_entries, tables begin at each lane's row.
        self.desc = np.zeros((lanes, self.max_entries), dtype=dev.BLOCK_DESC)
        for i in range(lanes):
            d = self.desc[i]
            d["slot"][: self.ext_per_lane] = ext_perm[i * self.ext_per_lane:(i + 1) * self.ext_per_lane]
            d["generation"][: self.ext_per_lane] = 1
            d["logical_token_begin"][: self.ext_per_lane] = np.arange(self.ext_per_lane) * 64
            d["valid_tokens"][: self.ext_per_lane] = 64
            d["page_token_capacity"][: self.ext_per_lane] = 64
            d["kind"][: self.ext_per_lane] = 1
            m = self.ext_per_lane
            d["slot"][m:] = micro_perm[i * self.micro_per_lane:(i + 1) * self.micro_per_lane]
            d["generation"][m:] = 1
            d["logical_token_begin"][m:] = context + np.arange(self.micro_per_lane) * 8
            d["page_token_capacity"][m:] = 8
            d["kind"][m:] = 0
        self.desc_dev = dev.upload(self.desc)
        self.desc_stride = self.max_entries * dev.BLOCK_DESC.itemsize
        # Fill every context page with the synthetic generator (stream id = lane).
        t0 = time.time()
        for i in range(lanes):
            self.storage.fill_table(self.desc_dev.ptr + i * self.desc_stride, self.ext_per_lane, 0, context,
                                    seed, i)
            if (i + 1) % 64 == 0:
                dev.sync()
                log(f"  filled {i + 1}/{lanes} lanes ({time.time() - t0:.1f}s)")
        dev.sync()
        log(f"filled {lanes} x {context} tokens in {time.time() - t0:.1f}s")
        # New K/V per (lane, layer, comp, step) and queries per (lane, layer, step).
        HD = kv_heads * head_dim
        self.newkv = dev.DeviceBuffer(lanes * layers * 2 * total_steps * HD * 2)
        self.query = dev.DeviceBuffer(lanes * layers * total_steps * query_heads * head_dim * 2)
        self.qseed = seed ^ 0x5155455259
        for i in range(lanes):
            for l in range(layers):
                for c in range(2):
                    off = (((i * layers + l) * 2 + c) * total_steps) * HD
                    dev.fill_rows(self.newkv.ptr + 2 * off, total_steps * HD, seed,
                                  dev.synth_kv_row(i, l, c, context), HD)
                qoff = ((i * layers + l) * total_steps) * query_heads * head_dim
                dev.fill_rows(self.query.ptr + 2 * qoff, total_steps * query_heads * head_dim, self.qseed,
                              dev.synth_kv_row(i, l, 0, context), query_heads * head_dim)
        dev.sync()
        self.out = dev.DeviceBuffer(layers * lanes * query_heads * head_dim * 2)
        self.items_dev = dev.DeviceBuffer(layers * lanes * dev.DECODE_ITEM.itemsize)
        self.jobs_dev = dev.DeviceBuffer(layers * lanes * dev.APPEND_JOB.itemsize)
        self.prefix_dev = dev.DeviceBuffer((lanes + 1) * 4)
        self.ws = None
        self.ws_stride = 0
        self.step_index = 0

    def lane_tokens(self, step):
        return self.context + step + 1

    def prepare_step(self, step):
        """Host metadata for one step: tail entries, decode items, append jobs."""
        dev = self.dev
        m = self.ext_per_lane + step // 8
        self.desc["valid_tokens"][:, m] = step % 8 + 1
        count = m + 1
        T = self.lane_tokens(step)
        chunk, prefix, total = self.storage.decode_plan([T] * self.lanes, self.QH)
        if self.decode_mode == "head_split":      # one chunk per lane, split over the four waves
            chunk = (T + 63) // 64 * 64 | dev.DECODE_HEAD_SPLIT
        elif self.decode_mode == "guided":
            chunk = dev.DECODE_GUIDED | 64
        if self.decode_mode != "plan":
            prefix = dev.chunk_prefix([T] * self.lanes, chunk, self.D)
            total = int(prefix[-1])
        ws_lane = dev.workspace_bytes(T, chunk, self.QH, self.D)
        if self.ws is None or ws_lane > self.ws_stride:
            self.ws_stride = max(ws_lane, 256)
            self.ws = dev.DeviceBuffer(self.ws_stride * self.lanes)
        HD = self.H * self.D
        QD = self.QH * self.D
        L, N, S = self.L, self.lanes, self.total_steps
        lane = np.arange(N, dtype=np.uint64)
        items = np.zeros((L, N), dtype=dev.DECODE_ITEM)
        jobs = np.zeros((L, N), dtype=dev.APPEND_JOB)
        for l in range(L):
            it = items[l]
            it["descriptors"] = self.desc_dev.ptr + lane * np.uint64(self.desc_stride)
            it["descriptor_count"] = count
            it["token_count"] = T
            it["layer"] = l
            it["query"] = self.query.ptr + 2 * (((lane * L + l) * S + step) * QD)
            it["workspace"] = (self.ws.ptr + lane * np.uint64(self.ws_stride)) if ws_lane else 0
            it["output"] = self.out.ptr + 2 * ((l * N + lane) * QD)
            it["attention_scale"] = 1.0 / math.sqrt(self.D)
            jb = jobs[l]
            kbase = ((lane * L + l) * 2) * S
            jb["src_key"] = self.newkv.ptr + 2 * ((kbase + step) * HD)
            jb["src_value"] = self.newkv.ptr + 2 * ((kbase + S + step) * HD)
            jb["layer_begin"] = l
            jb["layer_count"] = 1
            jb["token_count"] = 1
            jb["dst_slot"] = self.desc["slot"][:, m]
            jb["dst_kind"] = 0
            jb["dst_token"] = step % 8
        self.items_host = items
        self.jobs_host = jobs
        self.prefix = prefix
        self.plan = (chunk, total)

    def upload_step(self, stream):
        dev = self.dev
        dev.copy_to_device(self.desc_dev.ptr, self.desc, stream)
        dev.copy_to_device(self.items_dev.ptr, self.items_host, stream)
        dev.copy_to_device(self.jobs_dev.ptr, self.jobs_host, stream)
        dev.copy_to_device(self.prefix_dev.ptr, self.prefix, stream)

    def launch_step(self, stream):
        dev = self.dev
        lib = dev.lib()
        chunk, total = self.plan
        sh = ctypes.c_void_p(stream.handle)
        for l in range(self.L):
            dev.check(lib.kimkv_append_batch(self.storage.h,
                                             ctypes.c_void_p(self.jobs_dev.ptr + l * self.lanes * dev.APPEND_JOB.itemsize),
                                             self.lanes, 1, sh), "append")
            dev.check(lib.kimkv_paged_decode_batch(
                self.storage.h, ctypes.c_void_p(self.items_dev.ptr + l * self.lanes * dev.DECODE_ITEM.itemsize),
                ctypes.c_void_p(self.prefix_dev.ptr), self.lanes, total, chunk, self.QH, sh), "decode")

    def step(self, step, stream):
        self.prepare_step(step)
        self.upload_step(stream)
        self.launch_step(stream)


class EngineWorkload:
    """The same workload driven through the engine API (createHeterogeneous
    backend, per step: reserveToken for every lane, then per layer one
    writeLayerBatch and one attendLayerBatch over all lanes, then commit).
    Contexts are built with the bulk prefill append + promotion, so every
    page id comes from the manager's (permuted) pools."""

    def __init__(self, kimkv, dev, lanes, context, layers, kv_heads, head_dim, query_heads, total_steps, seed,
                 groups=2, group_streams=True):
        import importlib
        host = importlib.import_module(kimkv.__name__ + ".host")
        self.dev, self.host = dev, host
        self.lanes, self.context, self.L = lanes, context, layers
        self.H, self.D, self.QH = kv_heads, head_dim, query_heads
        self.total_steps = total_steps
        self.seed = seed
        assert context % 64 == 0
        self.ext_per_lane = context // 64
        HD = kv_heads * head_dim
        n_ext = lanes * self.ext_per_lane
        n_micro = 512 // 8 + 8 + lanes * ((total_steps + 7) // 8 + 1)
        T_max = context + total_steps
        self.ws_lane = max(dev.workspace_bytes(T_max, 64, query_heads, head_dim), 256)
        t0 = time.time()
        self.engine = host.Engine(layers, kv_heads, head_dim, query_heads, self.ws_lane, n_micro, n_ext)
        snap = self.engine.snapshot()
        log(f"engine pools: {snap.storage_reserved_bytes / 1e9:.1f} GB ({time.time() - t0:.1f}s)")
        t0 = time.time()
        for kind, sd in ((1, seed), (0, seed + 1)):
            rc = self.engine.permute_free_slots(kind, sd)
            if rc != 0:
                raise RuntimeError(f"permute_free_slots({kind}) failed: {host.ENGINE_ERRORS[rc]}")
        log(f"permuted free lists ({time.time() - t0:.1f}s)")
        # Prefill in 512-token chunks: synthetic [L][2][512][H][D] (stream id = lane),
        # bulk append, then promotion of the chunk's eight 64-token runs.
        chunk = 512
        stage = dev.DeviceBuffer(layers * 2 * chunk * HD * 2)
        stream = dev.Stream()
        t0 = time.time()
        for i in range(lanes):
            rc = self.engine.create_request(i + 1)
            assert rc == 0, host.ENGINE_ERRORS[rc]
            for t in range(0, context, chunk):
                dev.fill_kv(stage.ptr, layers, chunk, HD, seed, i, t, stream)
                rc, promoted = self.engine.append_prefill(i + 1, chunk, stage.ptr, stream, promote=True)
                if rc != 0 or promoted != chunk // 64:
                    raise RuntimeError(f"prefill lane {i} at {t}: {host.ENGINE_ERRORS[rc]}, promoted {promoted}")
            if (i + 1) % 64 == 0:
                log(f"  prefilled {i + 1}/{lanes} lanes ({time.time() - t0:.1f}s)")
        stream.synchronize()
        del stage
        log(f"prefilled {lanes} x {context} tokens in {time.time() - t0:.1f}s")
        # New K/V per (lane, layer, comp, step) and queries per (lane, layer, step), as in the kernel path.
        S = total_steps
        self.newkv = dev.DeviceBuffer(lanes * layers * 2 * S * HD * 2)
        self.query = dev.DeviceBuffer(lanes * layers * S * query_heads * head_dim * 2)
        self.qseed = seed ^ 0x5155455259
        for i in range(lanes):
            for l in range(layers):
                for c in range(2):
                    off = (((i * layers + l) * 2 + c) * S) * HD
                    dev.fill_rows(self.newkv.ptr + 2 * off, S * HD, seed, dev.synth_kv_row(i, l, c, context), HD)
                qoff = ((i * layers + l) * S) * query_heads * head_dim
                dev.fill_rows(self.query.ptr + 2 * qoff, S * query_heads * head_dim, self.qseed,
                              dev.synth_kv_row(i, l, 0, context), query_heads * head_dim)
        dev.sync()
        QD = query_heads * head_dim
        self.out = dev.DeviceBuffer(layers * lanes * QD * 2)
        self.ws = dev.DeviceBuffer(self.ws_lane * lanes)
        lane = np.arange(lanes, dtype=np.uint64)
        lay = np.arange(layers, dtype=np.uint64)[:, None]
        kbase = self.newkv.ptr + np.uint64(2 * HD) * ((lane[None, :] * np.uint64(layers) + lay) * np.uint64(2 * S))
        qbase = self.query.ptr + np.uint64(2 * QD) * ((lane[None, :] * np.uint64(layers) + lay) * np.uint64(S))
        obase = self.out.ptr + np.uint64(2 * QD) * (lay * np.uint64(lanes) + lane[None, :])
        # Lane groups: each group is one batch of token transactions; with two
        # groups the host reserves/launches one while the GPU runs the other.
        # With group_streams each group has its own stream, so one group's
        # decode launch fills the compute units that the other's last
        # workgroups leave idle at the end of a launch.
        self.groups = []
        self.streams = [stream]
        bounds = np.linspace(0, lanes, groups + 1).astype(int)
        for g in range(groups):
            sl = slice(bounds[g], bounds[g + 1])
            gs = stream
            if group_streams and g > 0:
                gs = dev.Stream()
                self.streams.append(gs)
            b = host.LaneBatch(self.engine, lane[sl] + np.uint64(1), self.ws.ptr + lane[sl] * np.uint64(self.ws_lane),
                               self.ws_lane, 1.0 / math.sqrt(head_dim), gs)
            b.outputs[:] = obase[:, sl]
            self.groups.append((b, kbase[:, sl], kbase[:, sl] + np.uint64(2 * HD * S), qbase[:, sl]))
        self.stream = stream
        self.reserve_s = 0.0
        self.commit_s = 0.0
        self.plan = (0, 0)
        self.pending = None

    def lane_tokens(self, step):
        return self.context + step + 1

    @staticmethod
    def _check(b, what):
        if b.failed():
            raise RuntimeError(f"{what}: {sorted(set(b.status.tolist()))}")

    def _launch(self, group, step):
        b, kb, vb, qb = group
        HD, QD = self.H * self.D, self.QH * self.D
        b.keys[:] = kb + np.uint64(2 * HD * step)
        b.values[:] = vb + np.uint64(2 * HD * step)
        b.queries[:] = qb + np.uint64(2 * QD * step)
        t0 = time.perf_counter()
        b.reserve(self.context + step)
        self.reserve_s += time.perf_counter() - t0
        self._check(b, "reserve")
        for l in range(self.L):
            b.write(l)
            self._check(b, f"writeLayerBatch layer {l}")
            b.attend(l)
            self._check(b, f"attendLayerBatch layer {l}")

    def _commit(self, group):
        b = group[0]
        t0 = time.perf_counter()
        b.commit()
        self.commit_s += time.perf_counter() - t0
        self._check(b, "commit")

    def step(self, step, stream=None):
        """One token for every lane.  A group is committed only after the next
        group's layers are queued, so the GPU has work while the host commits
        one group and reserves the next."""
        for g in self.groups:
            if self.pending is g:          # a single group commits before its next token
                self._commit(g)
                self.pending = None
            self._launch(g, step)
            if self.pending is not None:
                self._commit(self.pending)
            self.pending = g

    def drain(self):
        if self.pending is not None:
            self._commit(self.pending)
            self.pending = None


def cpu_baseline(kimkv, w: Workload, lanes_sample: int, step: int, threads: int):
    """Oracle decode of `lanes_sample` lanes x 1 layer at full context, timed
    once on one thread and once with the lanes spread over `threads` threads
    (the oracle's C decode runs without the GIL)."""
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    layer = 0
    T = w.lane_tokens(step)
    H, D, QH = w.H, w.D, w.QH
    cases = []
    for lane in range(lanes_sample):
        n_ext = w.ext_per_lane
        n_micro = (step // 8) + 1
        pools = oracle.HostPools(1, H, D, n_micro, n_ext)
        table = np.zeros(n_ext + n_micro, dtype=oracle.DESC)
        # Rebuild this lane's layer-0 KV from the generator into host pages (reference layout, L=1).
        kv = np.empty((1, 2, T, H, D), dtype=np.uint16)
        for c in range(2):
            rows = oracle.synth_rows(w.context * H * D, w.seed, oracle.kv_row(lane, layer, c, 0), H * D)
            kv[0, c, :w.context] = rows.reshape(w.context, H, D)
            new = oracle.synth_rows((step + 1) * H * D, w.seed, oracle.kv_row(lane, layer, c, w.context), H * D)
            kv[0, c, w.context:] = new.reshape(step + 1, H, D)
        for e in range(n_ext):
            table[e] = (e, 1, 64 * e, 64, 64, 1)
            pools.append_tokens(kv, T, 64 * e, 1, e, 0, 64)
        for k in range(n_micro):
            b = w.context + 8 * k
            n = min(8, T - b)
            table[n_ext + k] = (k, 1, b, n, 8, 0)
            pools.append_tokens(kv, T, b, 0, k, 0, n)
        q = oracle.synth_rows(QH * D, w.qseed, oracle.kv_row(lane, layer, 0, w.context) + step, QH * D)
        cases.append((pools, table, q))

    def decode(case):
        pools, table, q = case
        return pools.paged_decode(table, T, layer, QH, q, 1.0 / math.sqrt(D), f32=True)

    t0 = time.perf_counter()
    outs = [decode(c) for c in cases]
    serial_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as pool:
        par = list(pool.map(decode, cases))
    parallel_s = time.perf_counter() - t0
    for a, b in zip(outs, par):
        if not np.array_equal(a, b):
            raise RuntimeError("threaded oracle decode differs from the serial run")
    kv_bytes = lanes_sample * T * 2 * H * D * 2
    return outs, serial_s, parallel_s, kv_bytes


def run_gather(dev, args) -> int:
    """Long-sequence gather: one sequence of --gather-tokens tokens x 22 layers in
    64-token extents (permuted slots) -> contiguous [22][2][T][4][64].  Also the
    known-size copy used to calibrate the FETCH_SIZE / WRITE_SIZE counters."""
    L, H, D = args.layers, 4, 64
    T = args.gather_tokens
    n_ext = T // 64
    n_micro = (T % 64 + 7) // 8 + 1
    storage = dev.Storage(L, H, D, n_micro, n_ext)
    ext_perm = permutation(args.seed, n_ext)
    entries = [(int(ext_perm[e]), 1, 64 * e, 64, 64, 1) for e in range(n_ext)]
    b = 64 * n_ext
    k = 0
    while b < T:
        n = min(8, T - b)
        entries.append((k, 1, b, n, 8, 0))
        b += n
        k += 1
    table = np.array(entries, dtype=dev.BLOCK_DESC)
    d = dev.upload(table)
    storage.fill_table(d.ptr, len(table), 0, T, args.seed, 0)
    n = L * 2 * T * H * D
    out = dev.DeviceBuffer(n * 2)
    stream = dev.Stream()
    lib = dev.lib()
    sh = ctypes.c_void_p(stream.handle)

    def launch():
        dev.check(lib.kimkv_gather(storage.h, ctypes.c_void_p(d.ptr), len(table), T, ctypes.c_void_p(out.ptr), sh),
                  "gather")

    for _ in range(args.warmup):
        launch()
    stream.synchronize()
    start, stop = dev.Event(), dev.Event()
    start.record(stream)
    for _ in range(args.steps):
        launch()
    stop.record(stream)
    stop.synchronize()
    ms = start.elapsed_ms(stop) / args.steps
    moved = 2 * n * 2                       # read + write
    got = dev.download(out.ptr, (L, 2, T, H * D), np.uint16)
    # Bit-exact check of sampled (layer, component, token) rows against the generator.
    import oracle
    rng = np.random.default_rng(args.seed)
    bad = 0
    for _ in range(256):
        l, c, t = int(rng.integers(L)), int(rng.integers(2)), int(rng.integers(T))
        want = oracle.synth_rows(H * D, args.seed, oracle.kv_row(0, l, c, t), H * D)
        bad += int(not np.array_equal(got[l, c, t], want))
    cpu = cpu_gather_baseline(args, entries, T, L, H, D, moved) if args.cpu_lanes > 0 else None
    print(json.dumps({
        "metric": "long-sequence gather (paged -> contiguous) GB/s", "value": round(moved / (ms * 1e-3) / 1e9, 1),
        "unit": "GB/s", "us_per_launch": round(ms * 1000, 2), "bytes_per_launch": moved,
        "read_bytes": n * 2, "write_bytes": n * 2, "pct_of_peak_hbm": round(100 * moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
        "roofline": {"bound": "hbm", "achieved": round(moved / (ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("gather_kernel_long_sequence.md", tokens=T, layers=L),
                     "kernel": "gather_kernel", "launch_ms": round(ms, 4), "bytes_per_launch": moved},
        "config": {"workload": f"gather of one {T}-token sequence x {L} layers (4 kv heads x 64, fp16), "
                               f"{n_ext} extents in permuted slots + {k} micro pages"},
        "steps": args.steps, "check": {"sampled_rows": 256, "mismatches": bad}, "cpu_baseline": cpu_on_host(cpu)}), flush=True)
    return 0 if bad == 0 else 1


def synth_history(seed, stream_of, layers, T, H, D, threads):
    """[len(layers)][2][T][H][D] generator rows: token t is row kv_row(stream_of(t), layer, comp, t); the
    (layer, comp) blocks are generated on `threads` threads (the oracle's C calls release the GIL)."""
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    out = np.empty((len(layers), 2, T, H, D), dtype=np.uint16)
    runs, a = [], 0
    while a < T:
        sid, b = stream_of(a), a + 1
        while b < T and stream_of(b) == sid:
            b += 1
        runs.append((sid, a, b))
        a = b

    def fill(job):
        li, l, c = job
        for sid, a, b in runs:
            out[li, c, a:b] = oracle.synth_rows((b - a) * H * D, seed, oracle.kv_row(sid, l, c, a), H * D) \
                .reshape(b - a, H, D)

    with ThreadPoolExecutor(max_workers=threads) as pool:
        list(pool.map(fill, [(li, l, c) for li, l in enumerate(layers) for c in range(2)]))
    return out


def cpu_gather_baseline(args, entries, T, L, H, D, moved):
    """The oracle's gather of the same table (same slots, same generator rows), on one host core: the
    reference's CPU data path is single-threaded and the oracle gathers a table in one call."""
    import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
    kv = synth_history(args.seed, lambda t: 0, list(range(L)), T, H, D, threads)
    n_ext = sum(1 for e in entries if e[5] == 1)
    n_micro = max([e[0] for e in entries if e[5] == 0] + [0]) + 1
    pools = oracle.HostPools(L, H, D, n_micro, n_ext)
    table = np.array(entries, dtype=oracle.DESC)
    for slot, _, b, n, _, kind in entries:
        pools.append_tokens(kv, T, b, kind, slot, 0, n)
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        out = pools.gather(table, T)
    sec = (time.perf_counter() - t0) / reps
    if not np.array_equal(out, kv.reshape(-1)):
        raise RuntimeError("oracle gather differs from the generator")
    return {"value": round(moved / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "us_per_launch": round(sec * 1e6, 1),
            "sample": f"the whole workload: oracle kvo_gather of the same {T}-token x {L}-layer table, mean of "
                      f"{reps} calls on {host_cpu()['model']}",
            "seconds": round(sec * reps, 2)}


def run_append(kimkv, dev, args) -> int:
    """Ragged append: 64 lanes with contexts uniform in [1, 4096] tokens (seeded),
    22 layers x 4 kv heads x 64 fp16, micro/extent pages in permuted pool order
    (contexts built by bulk append + promotion of every full 64-token run).
    One step appends one token of K/V per lane per layer into the page tails,
    tail-page allocation (and its metadata) included: HipKvCache::appendBatch,
    i.e. per lane metadata append + leases, then one append kernel for all
    lanes and layers, waited for."""
    import importlib
    import oracle
    host = importlib.import_module(kimkv.__name__ + ".host")
    L, H, D = args.layers, 4, 64
    HD = H * D
    lanes = args.append_lanes
    rng = np.random.default_rng(args.seed)
    lengths = rng.integers(1, 4097, lanes)
    timing_steps = 8                       # after the timed loop: append kernel duration by events
    total_steps = args.warmup + args.steps + timing_steps
    n_ext = int(sum(lengths // 64)) + 16
    n_micro = 512 + lanes * (8 + total_steps // 8 + 2)
    cache = host.Cache(L, H, D, n_micro, n_ext)
    for kind, sd in ((1, args.seed), (0, args.seed + 1)):
        rc = cache.permute_free_slots(kind, sd)
        assert rc == 0, rc
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * 4096 * HD * 2)
    t0 = time.time()
    for i in range(lanes):
        assert cache.create_request(i + 1) == 0
        n = int(lengths[i])
        dev.fill_kv(stage.ptr, L, n, HD, args.seed, i, 0, stream)
        r = cache.append(i + 1, n, stage.ptr, stream)
        assert r.ok(), (r.metadata_error, r.device_status)
        for b in range(0, n - n % 64, 64):
            r = cache.promote(i + 1, b, stream)
            assert r.ok(), (i, b, r.metadata_error, r.device_status)
    log(f"built {lanes} contexts ({int(lengths.sum())} tokens) in {time.time() - t0:.1f}s")
    # New token per (lane, step): [L][2][1][HD] blocks, rows kv_row(lane, l, c, length + step).
    per = L * 2 * HD
    newkv = dev.DeviceBuffer(lanes * total_steps * per * 2)
    for i in range(lanes):
        for s_ in range(total_steps):
            dev.fill_kv(newkv.ptr + 2 * (i * total_steps + s_) * per, L, 1, HD, args.seed, i,
                        int(lengths[i]) + s_, stream)
    stream.synchronize()
    ids = np.arange(1, lanes + 1, dtype=np.uint64)
    results = (host.CacheResult * lanes)()
    lane = np.arange(lanes, dtype=np.uint64)

    # Every step's input addresses, computed before the timed loop.
    steps_in = [newkv.ptr + np.uint64(2 * per) * (lane * np.uint64(total_steps) + np.uint64(t))
                for t in range(total_steps)]

    # The results as one int32 pair per lane (metadata error, device
    # status): every lane is checked in one vector test.
    res_words = np.frombuffer(results, dtype=np.int32)

    def step(s_):
        cache.append_batch(ids, 1, steps_in[s_], results, stream)
        if res_words.any():
            bad = [k for k in range(lanes) if not results[k].ok()]
            raise RuntimeError(f"append failed for lanes {bad[:4]}: {results[bad[0]].metadata_error}, "
                               f"{results[bad[0]].device_status}")

    for s_ in range(args.warmup):
        step(s_)
    start, stop = dev.Event(), dev.Event()
    walls = []
    start.record(stream)
    for s_ in range(args.warmup, args.warmup + args.steps):
        t = time.perf_counter()
        step(s_)
        walls.append(time.perf_counter() - t)
    stop.record(stream)
    stop.synchronize()
    gpu_ms = start.elapsed_ms(stop)
    dev.append_timing(True)
    for s_ in range(args.warmup + args.steps, total_steps):
        step(s_)
    stream.synchronize()
    ap_ms, ap_n = dev.append_timing(False)
    wall_us = 1e6 * sum(walls) / len(walls)
    step_bytes = lanes * L * 2 * (2 * HD * 2)          # read new K/V + write into the page
    # Bit-exact check: gather sampled lanes and compare with the generator.
    bad = 0
    checked = 0
    for i in rng.choice(lanes, size=min(args.append_check, lanes), replace=False):
        T = int(lengths[i]) + total_steps
        out = dev.DeviceBuffer(L * 2 * T * HD * 2)
        r = cache.gather(int(i) + 1, out.ptr, stream)
        assert r.ok()
        got = dev.download(out.ptr, (L, 2, T, HD), np.uint16, stream)
        for l in range(L):
            for c in range(2):
                want = oracle.synth_rows(T * HD, args.seed, oracle.kv_row(int(i), l, c, 0), HD).reshape(T, HD)
                bad += int(not np.array_equal(got[l, c], want))
        checked += 1
    # CPU baseline: the same step's page writes by the oracle (one
    # kvo_append_tokens call per lane writes its token in all layers).
    pools = oracle.HostPools(L, H, D, lanes, 1)
    steps_cpu = 200
    newrows = np.empty((lanes, L, 2, 1, H, D), dtype=np.uint16)
    for i in range(lanes):
        for l in range(L):
            for c in range(2):
                newrows[i, l, c, 0] = oracle.synth_rows(HD, args.seed, oracle.kv_row(i, l, c, int(lengths[i])),
                                                        HD).reshape(H, D)
    t0 = time.perf_counter()
    for s_ in range(steps_cpu):
        for i in range(lanes):
            pools.append_tokens(newrows[i], 1, 0, 0, i, s_ % 8, 1)
    cpu_us = (time.perf_counter() - t0) * 1e6 / steps_cpu
    cpu = {"value": round(cpu_us, 2), "unit": "us/step", "cores": 1, "kind": "port",
           "gb_per_s": round(step_bytes / (cpu_us * 1e-6) / 1e9, 3),
           "sample": f"{steps_cpu} steps of {lanes} oracle kvo_append_tokens calls (1 token x {L} layers each) through "
                     f"ctypes on {host_cpu()['model']}; page writes only, the page-table "
                     f"metadata is this library's host code in both runs"}
    print(json.dumps({
        "metric": "ragged KV append (1 token x 22 layers per lane, tail allocation included) us/step",
        "value": round(wall_us, 2), "unit": "us/step", "higher_is_better": False,
        "gb_per_s": round(step_bytes / (wall_us * 1e-6) / 1e9, 2), "bytes_per_step": step_bytes,
        "gpu_span_us_per_step": round(1000 * gpu_ms / args.steps, 2),
        "append_kernel_avg_us": round(1000 * ap_ms / max(ap_n, 1), 2),
        "roofline": {"bound": "hbm", "achieved": round(step_bytes / (ap_ms / max(ap_n, 1) * 1e-3) / 1e9, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(step_bytes / (ap_ms / max(ap_n, 1) * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("append_kernel_ragged_append.md", lanes=lanes, layers=L),
                     "kernel": "append_kernel", "launch_ms": round(ap_ms / max(ap_n, 1), 4),
                     "timed_launches": ap_n, "bytes_per_launch": step_bytes,
                     "note": f"latency-bound: one launch of {lanes * L} (lane, layer) jobs of 1 KiB K + 1 KiB V each"},
        "config": {"workload": f"{lanes} lanes, contexts uniform in [1, 4096] tokens, {L} layers x 4 kv heads x 64 "
                               f"fp16, micro/extent pages in permuted pool order",
                   "tokens": int(lengths.sum())},
        "steps": args.steps, "warmup": args.warmup,
        "check": {"lanes": checked, "mismatched_rows_blocks": bad, "bit_exact": bad == 0},
        "cpu_baseline": cpu_on_host(cpu)}), flush=True)
    return 0 if bad == 0 else 1


def run_parity(kimkv, dev, args) -> int:
    """Config 1: one TinyLlama layer (32 q / 4 kv heads x 64, fp16), 4 lanes with
    contexts {17, 100, 513, 1000} built by bulk prefill + promotion in
    512-slot micro and extent pools with seeded permuted slots.  One step =
    reserve one token per lane, write its K/V, decode all 32 query heads
    (scale 1/8), commit, through the engine's batch API.  Latency-bound: the
    value is microseconds per step; the oracle's decode of the same 4 lanes
    is the CPU baseline."""
    import importlib
    import oracle
    host = importlib.import_module(kimkv.__name__ + ".host")
    L, H, D, QH = 1, 4, 64, 32
    HD, QD = H * D, QH * D
    contexts = [17, 100, 513, 1000]
    lanes = len(contexts)
    timing_steps = 20                      # after the timed loop: decode kernel duration by events
    total_steps = args.warmup + args.steps + timing_steps
    ws_lane = max(dev.workspace_bytes(max(contexts) + total_steps, 64, QH, D), 256)
    engine = host.Engine(L, H, D, QH, ws_lane, 512, 512)
    for kind, sd in ((1, args.seed), (0, args.seed + 1)):
        assert engine.permute_free_slots(kind, sd) == 0
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * max(contexts) * HD * 2)
    for i, T in enumerate(contexts):
        assert engine.create_request(i + 1) == 0
        dev.fill_kv(stage.ptr, L, T, HD, args.seed, i, 0, stream)
        rc, _ = engine.append_prefill(i + 1, T, stage.ptr, stream, promote=True)
        assert rc == 0, host.ENGINE_ERRORS[rc]
    S = total_steps
    newkv = dev.DeviceBuffer(lanes * 2 * S * HD * 2)
    query = dev.DeviceBuffer(lanes * S * QD * 2)
    out = dev.DeviceBuffer(lanes * QD * 2)
    qseed = args.seed ^ 0x51
    for i, T in enumerate(contexts):
        for c in range(2):
            dev.fill_rows(newkv.ptr + 2 * ((i * 2 + c) * S * HD), S * HD, args.seed, dev.synth_kv_row(i, 0, c, T), HD)
        dev.fill_rows(query.ptr + 2 * (i * S * QD), S * QD, qseed, dev.synth_kv_row(i, 0, 0, T), QD)
    lane = np.arange(lanes, dtype=np.uint64)
    ws = dev.DeviceBuffer(lanes * ws_lane)
    b = host.LaneBatch(engine, lane + np.uint64(1), ws.ptr + lane * np.uint64(ws_lane), ws_lane, 0.125, stream)
    b.outputs[0, :] = out.ptr + np.uint64(2 * QD) * lane
    stream.synchronize()

    # Every step's input addresses and expected lengths, computed before the
    # timed loop (the step copies them into the batch's argument arrays).
    steps_k = [newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * S) + np.uint64(t)) for t in range(S)]
    steps_v = [newkv.ptr + np.uint64(2 * HD) * (lane * np.uint64(2 * S) + np.uint64(S + t)) for t in range(S)]
    steps_q = [query.ptr + np.uint64(2 * QD) * (lane * np.uint64(S) + np.uint64(t)) for t in range(S)]
    steps_e = [np.array(contexts, dtype=np.uint32) + np.uint32(t) for t in range(S)]

    def step(s_):
        b.keys[0, :] = steps_k[s_]
        b.values[0, :] = steps_v[s_]
        b.queries[0, :] = steps_q[s_]
        b.reserve(steps_e[s_])
        b.write(0)
        b.attend(0)
        b.commit()
        assert not b.failed(), b.status

    for s_ in range(args.warmup):
        step(s_)
    t0 = time.perf_counter()
    for s_ in range(args.warmup, args.warmup + args.steps):
        step(s_)
    us = (time.perf_counter() - t0) * 1e6 / args.steps
    dev.decode_timing(True)
    for s_ in range(args.warmup + args.steps, total_steps):
        step(s_)
    stream.synchronize()
    dec_ms, dec_n = dev.decode_timing(False)
    dec_ms /= max(dec_n, 1)
    # Algorithmic bytes of one decode launch: every lane's K/V (mean over the
    # timed launches) plus the queries, the outputs and the tokens written.
    mean_ctx = sum(contexts) + lanes * (args.warmup + args.steps + (timing_steps + 1) / 2.0)
    dec_bytes = mean_ctx * 2 * HD * 2 + lanes * (2 * QD * 2 + 2 * HD * 2)
    got = dev.download(out.ptr, (lanes, QD), np.uint16)
    # Oracle: the last step of every lane (history regenerated), timed on one core.
    last = total_steps - 1
    cases = []
    for i, T0 in enumerate(contexts):
        T = T0 + last + 1
        kv = synth_history(args.seed, lambda t, i=i: i, [0], T, H, D, 1)
        q = oracle.synth_rows(QD, qseed, oracle.kv_row(i, 0, 0, T0) + last, QD)
        cases.append((oracle_pages_layer(kv[0], T), T, q))
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        refs = [pools.paged_decode(table, T, 0, QH, q, 0.125, f32=True) for (pools, table), T, q in cases]
    cpu_us = (time.perf_counter() - t0) * 1e6 / reps
    worst, ok = 0.0, True
    for i, ref in enumerate(refs):
        err = np.abs(got[i].view(np.float16).astype(np.float32) - ref)
        worst = max(worst, float(err.max()))
        ok = ok and bool(np.all(err <= 2e-3 + 1e-3 * np.abs(ref)))
    assert engine.check_invariants()
    print(json.dumps({
        "metric": "config-1 decode step (reserve + write + GQA decode + commit, 4 lanes, 1 layer) us/step",
        "value": round(us, 2), "unit": "us/step", "higher_is_better": False,
        "config": {"workload": "one TinyLlama layer, 4 lanes, contexts 17/100/513/1000 (+1 appended per step), "
                               "512-slot permuted micro/extent pools, through the engine"},
        "steps": args.steps, "warmup": args.warmup,
        "check": {"lanes": lanes, "max_abs_err": worst, "within_tolerance": ok, "tolerance": "2e-3 + 1e-3*|ref|"},
        "decode_kernel_avg_us": round(dec_ms * 1000, 2),
        "roofline": {"bound": "hbm", "achieved": round(dec_bytes / (dec_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dec_bytes / (dec_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("decode_kernel_config1_step.md", lanes=lanes, layers=L),
                     "kernel": "decode_kernel", "launch_ms": round(dec_ms, 4),
                     "timed_launches": dec_n, "bytes_per_launch": int(dec_bytes),
                     "note": "latency-bound: 4 lanes, 1.6 k tokens of K/V in one launch"},
        "cpu_baseline": cpu_on_host({"value": round(cpu_us, 1), "unit": "us/step", "cores": 1, "kind": "port",
                         "sample": f"the decode of the whole step: oracle kvo_paged_decode of the 4 lanes, mean of "
                                   f"{reps} on {host_cpu()['model']}"})}), flush=True)
    return 0 if ok else 1


def oracle_pages_layer(kv_layer, T):
    """Host pages (8-token micro pages, one layer) holding kv_layer [2][T][H][D] and their table."""
    import oracle
    H, D = kv_layer.shape[2], kv_layer.shape[3]
    pages = (T + 7) // 8
    pools = oracle.HostPools(1, H, D, pages, 1)
    table = np.zeros(pages, dtype=oracle.DESC)
    kv = np.ascontiguousarray(kv_layer[None])
    for k in range(pages):
        n = min(8, T - 8 * k)
        table[k] = (k, 1, 8 * k, n, 8, 0)
        pools.append_tokens(kv, T, 8 * k, 0, k, 0, n)
    return pools, table


def oracle_decode_layer(kv_layer, T, q, QH, D):
    """fp32-accumulated GQA decode of one layer (kv_layer: uint16 [2][T][H][D]) by the oracle, with the
    tokens held in 8-token pages (the page structure does not change the result)."""
    import oracle
    H = kv_layer.shape[2]
    n_pages = (T + 7) // 8
    pools = oracle.HostPools(1, H, D, n_pages, 1)
    kv = kv_layer.reshape(1, 2, T, H, D)
    table = np.zeros(n_pages, dtype=oracle.DESC)
    for k in range(n_pages):
        b = 8 * k
        n = min(8, T - b)
        table[k] = (k, 1, b, n, 8, 0)
        pools.append_tokens(kv, T, b, 0, k, 0, n)
    return pools.paged_decode(table, T, 0, QH, q, 1.0 / math.sqrt(D), f32=True)


def run_shared(kimkv, dev, args) -> int:
    """Batched paged decode with sharing: 32 lanes in 8 groups of 4, context
    lengths log-uniform in [128, 8192] (seeded).  Each group's root holds a
    2048 + r token prefix (r in 1..7, so the prefix ends in a partial micro
    page), the 4 lanes fork it, and each lane's first own token copies that
    partial page (copy-on-write) before the lanes diverge; lengths below the
    prefix are raised to prefix + 8.  Contexts are built through the engine
    (bulk prefill + promotion); one step = reserve 32 tokens, 22 x
    (writeLayerBatch + attendLayerBatch), commit."""
    import importlib
    host = importlib.import_module(kimkv.__name__ + ".host")
    L, H, D, QH = args.layers, 4, 64, 32
    HD, QD = H * D, QH * D
    groups, per_group = 8, 4
    lanes = groups * per_group
    rng = np.random.default_rng(args.seed)
    r = rng.integers(1, 8, groups)
    prefix = 2048 + r
    lengths = np.exp(rng.uniform(np.log(128), np.log(8192), lanes)).astype(np.int64)
    for g in range(groups):
        sl = slice(g * per_group, (g + 1) * per_group)
        lengths[sl] = np.maximum(lengths[sl], prefix[g] + 8)
    total_steps = args.warmup + args.steps + 2      # + 2 steps with kernel timing
    n_ext = int(sum(lengths // 64)) + groups * 2 + 16
    n_micro = 1024 + lanes * (8 + total_steps // 8 + 2)
    ws_lane = max(dev.workspace_bytes(int(lengths.max()) + total_steps, 64, QH, D), 256)
    engine = host.Engine(L, H, D, QH, ws_lane, n_micro, n_ext)
    for kind, sd in ((1, args.seed), (0, args.seed + 1)):
        assert engine.permute_free_slots(kind, sd) == 0
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * int(lengths.max()) * HD * 2)
    root_sid = 200
    t0 = time.time()
    for g in range(groups):
        root = 10_000 + g
        assert engine.create_request(root) == 0
        P = int(prefix[g])
        dev.fill_kv(stage.ptr, L, P, HD, args.seed, root_sid + g, 0, stream)
        rc, _ = engine.append_prefill(root, P, stage.ptr, stream, promote=True)
        assert rc == 0, host.ENGINE_ERRORS[rc]
        for j in range(per_group):
            lane = g * per_group + j
            assert engine.fork_request(root, lane + 1) == 0
            n = int(lengths[lane]) - P
            dev.fill_kv(stage.ptr, L, n, HD, args.seed, lane, P, stream)
            rc, _ = engine.append_prefill(lane + 1, n, stage.ptr, stream, promote=True)
            assert rc == 0, host.ENGINE_ERRORS[rc]
        assert engine.release_request(root) == 0
    assert engine.check_invariants()
    log(f"built {lanes} shared contexts ({int(lengths.sum())} tokens) in {time.time() - t0:.1f}s")
    # Unique physical pages vs logical tokens (per layer).
    logical = int(lengths.sum())
    unique = {}
    for lane in range(lanes):
        _, entries = engine.block_table(lane + 1)
        for (b, v, k, slot, gen) in entries:
            unique[(k, slot)] = v
    physical = sum(unique.values())
    # Per-step inputs: new K/V rows kv_row(lane, l, c, length + step), queries.
    S = total_steps
    newkv = dev.DeviceBuffer(lanes * L * 2 * S * HD * 2)
    query = dev.DeviceBuffer(lanes * L * S * QD * 2)
    qseed = args.seed ^ 0x5155455259
    for i in range(lanes):
        for l in range(L):
            for c in range(2):
                off = (((i * L + l) * 2 + c) * S) * HD
                dev.fill_rows(newkv.ptr + 2 * off, S * HD, args.seed, dev.synth_kv_row(i, l, c, int(lengths[i])), HD)
            qoff = ((i * L + l) * S) * QD
            dev.fill_rows(query.ptr + 2 * qoff, S * QD, qseed, dev.synth_kv_row(i, l, 0, int(lengths[i])), QD)
    out = dev.DeviceBuffer(L * lanes * QD * 2)
    ws = dev.DeviceBuffer(ws_lane * lanes)
    lane_ix = np.arange(lanes, dtype=np.uint64)
    lay = np.arange(L, dtype=np.uint64)[:, None]
    kbase = newkv.ptr + np.uint64(2 * HD) * ((lane_ix[None, :] * np.uint64(L) + lay) * np.uint64(2 * S))
    vbase = kbase + np.uint64(2 * HD * S)
    qbase = query.ptr + np.uint64(2 * QD) * ((lane_ix[None, :] * np.uint64(L) + lay) * np.uint64(S))
    obase = out.ptr + np.uint64(2 * QD) * (lay * np.uint64(lanes) + lane_ix[None, :])
    # Lane groups (whole fork groups): one batch of token transactions each,
    # on its own stream, pipelined like the HBM-scale workload's groups (a
    # group commits after the next group's layers are queued).  One group
    # (the default) is the whole step as a single batch.
    n_groups = max(1, min(args.shared_groups, groups))
    bounds = [per_group * (groups * g // n_groups) for g in range(n_groups + 1)]
    streams = [stream] + [dev.Stream() for _ in range(n_groups - 1)]
    # Per group: its batch and every step's input addresses and expected
    # lengths, computed before the timed loop (a step copies them into the
    # batch's argument arrays).
    batches = []
    for g in range(n_groups):
        sl = slice(bounds[g], bounds[g + 1])
        b = host.LaneBatch(engine, lane_ix[sl] + np.uint64(1), ws.ptr + lane_ix[sl] * np.uint64(ws_lane), ws_lane,
                           1.0 / math.sqrt(D), streams[g])
        b.outputs[:] = obase[:, sl]
        batches.append((b, [np.ascontiguousarray(kbase[:, sl] + np.uint64(2 * HD * t)) for t in range(S)],
                        [np.ascontiguousarray(vbase[:, sl] + np.uint64(2 * HD * t)) for t in range(S)],
                        [np.ascontiguousarray(qbase[:, sl] + np.uint64(2 * QD * t)) for t in range(S)],
                        [(lengths[sl] + t).astype(np.uint32) for t in range(S)]))
    stream.synchronize()
    pending = []

    def commit(b):
        b.commit()
        assert not b.failed(), b.status

    def step(s_):
        for g in batches:
            b, ks, vs, qs, es = g
            if pending and pending[0] is g:   # a single group commits before its next token
                commit(pending.pop()[0])
            b.keys[:] = ks[s_]
            b.values[:] = vs[s_]
            b.queries[:] = qs[s_]
            b.reserve(es[s_])
            assert not b.failed(), b.status
            for l in range(L):
                b.write(l)
                assert not b.failed(), b.status
                b.attend(l)
                assert not b.failed(), b.status
            if pending:
                commit(pending.pop()[0])
            pending.append(g)

    def drain():
        while pending:
            commit(pending.pop()[0])
        for st in streams:
            st.synchronize()

    for s_ in range(args.warmup):
        step(s_)
    drain()
    # Timed loop without per-launch kernel timing (its events sit between the
    # kernels and lengthen a step of short launches).
    start, stop = dev.Event(), dev.Event()
    t_wall = time.perf_counter()
    start.record(stream)
    for s_ in range(args.warmup, args.warmup + args.steps):
        step(s_)
    drain()
    stop.record(stream)
    stop.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1000.0
    gpu_ms = start.elapsed_ms(stop)
    ms_per_step = max(gpu_ms, wall_ms) / args.steps
    # Decode kernel duration from a separate short loop with event timing.
    dev.decode_timing(True)
    for s_ in range(args.warmup + args.steps, total_steps):
        step(s_)
    drain()
    dec_total_ms, dec_n = dev.decode_timing(False)
    dec_busy_ms = dev.decode_timing_busy()
    dec_avg_ms = dec_total_ms / max(dec_n, 1)
    # Per launch: its share of the time the decode kernel occupied the GPU
    # (with several lane groups two launches overlap: the busy union over
    # the launches; one group: their mean duration).
    dec_ms = dec_busy_ms / max(dec_n, 1) if n_groups > 1 else dec_avg_ms
    # Algorithmic bytes of one decode launch (mean over the timed launches,
    # one per layer per group): the lanes' logical K/V, the queries, the
    # outputs and the tokens written.
    dec_appended = args.warmup + args.steps + (total_steps - args.warmup - args.steps + 1) / 2.0
    dec_bytes = ((lengths.sum() + lanes * dec_appended) * 2 * HD * 2 + lanes * (2 * QD * 2 + 2 * HD * 2)) / n_groups
    us_per_layer = ms_per_step * 1000.0 / L
    appended = args.warmup + (args.steps + 1) / 2.0          # mean tokens appended by the timed steps
    logical_bytes = (lengths.sum() + lanes * appended) * 2 * HD * 2
    physical_bytes = (physical + lanes * appended) * 2 * HD * 2
    # Check and CPU baseline: the last step's layer 0 of every lane by the
    # oracle (one host core, then the lanes over all cores), the GPU's
    # outputs against it.
    last = total_steps - 1
    got = dev.download(out.ptr, (lanes, QD), np.uint16)
    worst, ok = 0.0, True
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    threads = max(1, min(16, os.cpu_count() or 1))
    cases = []
    for i in range(lanes):
        g = i // per_group
        P = int(prefix[g])
        T = int(lengths[i]) + last + 1
        kv = synth_history(args.seed, lambda t, g=g, i=i, P=P: root_sid + g if t < P else i, [0], T, H, D, threads)
        q = oracle.synth_rows(QD, qseed, oracle.kv_row(i, 0, 0, int(lengths[i])) + last, QD)
        cases.append((oracle_pages_layer(kv[0], T), T, q))

    def decode(case):
        (pools, table), T, q = case
        return pools.paged_decode(table, T, 0, QH, q, 1.0 / math.sqrt(D), f32=True)

    t0 = time.perf_counter()
    refs = [decode(c) for c in cases]
    cpu_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as pool:
        par = list(pool.map(decode, cases))
    cpu_par_s = time.perf_counter() - t0
    for i, ref in enumerate(refs):
        assert np.array_equal(ref, par[i])
        a = got[i].view(np.float16).astype(np.float32)
        err = np.abs(a - ref)
        worst = max(worst, float(err.max()))
        ok = ok and bool(np.all(err <= 2e-3 + 1e-3 * np.abs(ref)))
    layer_bytes = sum(T for (_, T, _) in cases) * 2 * HD * 2
    cpu = {"value": round(cpu_s * 1e6, 1), "unit": "us/layer", "cores": 1, "kind": "port",
           "gb_per_s": round(layer_bytes / cpu_s / 1e9, 4),
           "sample": f"the whole layer: oracle kvo_paged_decode of all {lanes} lanes (layer 0, last step) on "
                     f"{host_cpu()['model']}",
           "seconds": round(cpu_s, 2),
           "all_cores": {"value": round(cpu_par_s * 1e6, 1), "unit": "us/layer", "cores": threads,
                         "gb_per_s": round(layer_bytes / cpu_par_s / 1e9, 4), "seconds": round(cpu_par_s, 2)}}
    print(json.dumps({
        "metric": "shared-prefix paged decode attn+append us/layer (logical GB/s)",
        "value": round(us_per_layer, 2), "unit": "us/layer", "higher_is_better": False,
        "logical_gb_per_s": round(logical_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "physical_gb_per_s": round(physical_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "decode_kernel_avg_us": round(1000 * dec_avg_ms, 2),
        "decode_busy_us_per_launch": round(1000 * dec_ms, 2),
        "ms_per_step": round(ms_per_step, 3),
        "gpu_ms_per_step": round(gpu_ms / args.steps, 3), "host_ms_per_step": round(wall_ms / args.steps, 3),
        "roofline": {"bound": "hbm", "achieved": round(dec_bytes / (dec_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dec_bytes / (dec_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("decode_kernel_shared_prefix.md", lanes=lanes // n_groups,
                                                 layers=L, logical_tokens=int(logical)),
                     "kernel": "decode_kernel", "launch_ms": round(dec_ms, 4), "timed_launches": dec_n,
                     "bytes_per_launch": int(dec_bytes),
                     "note": "bytes are the lanes' logical K/V; the fork groups share prefix pages, so the unique "
                             "pages are about half of them; latency-bound (one round of 256-token chunks); with "
                             "several lane groups two groups' launches overlap and launch_ms is the busy union "
                             "per launch"},
        "config": {"workload": f"{lanes} lanes ({groups} groups of {per_group} forking a 2048+r-token prefix, "
                               f"partial-tail COW), contexts log-uniform in [128, 8192], {L} layers TinyLlama GQA "
                               f"32q/4kv/64d fp16, through the engine"
                               + (f", as {n_groups} batches of {lanes // n_groups} lanes pipelined on "
                                  f"{n_groups} streams" if n_groups > 1 else ""),
                   "logical_tokens": logical, "unique_physical_tokens": physical,
                   "lane_groups": n_groups, "lanes_per_batch": lanes // n_groups},
        "steps": args.steps, "warmup": args.warmup,
        "check": {"lanes": lanes, "layer": 0, "max_abs_err": worst, "within_tolerance": ok,
                  "tolerance": "2e-3 + 1e-3*|ref|"},
        "cpu_baseline": cpu_on_host(cpu)}), flush=True)
    return 0 if ok else 1


PEAK_MFMA_F16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA


def run_prefill(kimkv, dev, args) -> int:
    """Chunked prefill through the engine: --prefill-lanes requests whose
    contexts hold T0 ~ U[256, 2048] (seeded) prompt tokens take one
    --prefill-chunk-token chunk each per step.  Each step forks every base
    request (the fork's partial tail is copied on write), then per layer one
    batched K/V write and one batched causal GQA prefill-attention launch for
    all chunks, finishes the chunks and releases the forks, so every step does
    the same work.  Roofline: attention FLOPs per launch (4 * QH * D per
    (query, visible key) pair) over the prefill kernel's event-timed duration,
    against dense fp16 MFMA peak."""
    import importlib
    host = importlib.import_module(kimkv.__name__ + ".host")
    L, H, D, QH = args.layers, 4, 64, 32
    HD, QD = H * D, QH * D
    lanes, n = args.prefill_lanes, args.prefill_chunk
    rng = np.random.default_rng(args.seed)
    T0 = rng.integers(256, 2049, lanes)
    if args.prefill_context:
        T0[:] = args.prefill_context
    total_steps = args.warmup + args.steps
    n_ext = int(sum((T0 + n) // 64)) * 2 + 16
    n_micro = 1024 + lanes * (n // 8 + 4) * 2
    engine = host.Engine(L, H, D, QH, 1 << 16, n_micro, n_ext)
    for kind, sd in ((1, args.seed), (0, args.seed + 1)):
        assert engine.permute_free_slots(kind, sd) == 0
    stream = dev.Stream()
    stage = dev.DeviceBuffer(L * 2 * int(T0.max()) * HD * 2)
    for i in range(lanes):
        assert engine.create_request(i + 1) == 0
        dev.fill_kv(stage.ptr, L, int(T0[i]), HD, args.seed, i, 0, stream)
        rc, _ = engine.append_prefill(i + 1, int(T0[i]), stage.ptr, stream, promote=True)
        assert rc == 0, host.ENGINE_ERRORS[rc]
    # Chunk inputs: K/V [lane][L][2][n][HD] (rows kv_row(lane, l, c, T0 + t)), queries [lane][L][n][QD].
    kv = dev.DeviceBuffer(lanes * L * 2 * n * HD * 2)
    q = dev.DeviceBuffer(lanes * L * n * QD * 2)
    out = dev.DeviceBuffer(lanes * L * n * QD * 2)
    qseed = args.seed ^ 0x5155455259
    for i in range(lanes):
        dev.fill_kv(kv.ptr + i * L * 2 * n * HD * 2, L, n, HD, args.seed, i, int(T0[i]), stream)
        for l in range(L):
            dev.fill_rows(q.ptr + ((i * L + l) * n * QD) * 2, n * QD, qseed, dev.synth_kv_row(i, l, 0, 0), QD)
    stream.synchronize()
    scale = 1.0 / math.sqrt(D)

    def kv_ptr(i, l, c):
        return kv.ptr + (((i * L + l) * 2 + c) * n * HD) * 2

    def step(s_):
        base = 1000 * (s_ + 1)
        chunks = []
        for i in range(lanes):
            assert engine.fork_request(i + 1, base + i) == 0
            rc, c = engine.prefill_begin(base + i, int(T0[i]), n, stream)
            assert rc == 0, host.ENGINE_ERRORS[rc]
            chunks.append(c)
        for l in range(L):
            st = host.prefill_write_batch(chunks, l, [kv_ptr(i, l, 0) for i in range(lanes)],
                                          [kv_ptr(i, l, 1) for i in range(lanes)])
            assert st == [0] * lanes, st
            st = host.prefill_attend_batch(chunks, l, [q.ptr + ((i * L + l) * n * QD) * 2 for i in range(lanes)],
                                           [out.ptr + ((i * L + l) * n * QD) * 2 for i in range(lanes)], scale)
            assert st == [0] * lanes, st
        for i, c in enumerate(chunks):
            assert c.finish() == 0
            c.close()
            assert engine.release_request(base + i) == 0

    for s_ in range(args.warmup):
        step(s_)
    stream.synchronize()
    start, stop = dev.Event(), dev.Event()
    dev.prefill_timing(True)
    t_wall = time.perf_counter()
    start.record(stream)
    for s_ in range(args.warmup, total_steps):
        step(s_)
    stop.record(stream)
    stop.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1000.0
    pf_ms, pf_n = dev.prefill_timing(False)
    ms_per_step = max(start.elapsed_ms(stop), wall_ms) / args.steps
    kernel_ms = pf_ms / max(pf_n, 1)
    pairs = float(sum(n * int(t) + n * (n + 1) // 2 for t in T0))     # (query, visible key) pairs per layer
    flops = 4.0 * QH * D * pairs
    kv_bytes = float(sum(int(t) + n for t in T0)) * 2 * HD * 2 + 2 * lanes * n * QD * 2
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    # Check sampled rows of layers 0 and L-1 against the oracle's decode of
    # the first T0 + r + 1 tokens; the oracle's decode of those rows is also
    # the CPU baseline (one core), as FLOP/s over the same per-pair count.
    import oracle
    worst, ok, rows = 0.0, True, 0
    cpu_s, cpu_pairs = 0.0, 0
    for i in range(lanes):
        t0 = int(T0[i])
        for l in (0, L - 1):
            kvl = np.empty((2, t0 + n, H, D), dtype=np.uint16)
            for c in range(2):
                kvl[c, :t0] = oracle.synth_rows(t0 * HD, args.seed, oracle.kv_row(i, l, c, 0), HD).reshape(t0, H, D)
                kvl[c, t0:] = oracle.synth_rows(n * HD, args.seed, oracle.kv_row(i, l, c, t0), HD).reshape(n, H, D)
            ql = oracle.synth_rows(n * QD, qseed, oracle.kv_row(i, l, 0, 0), QD).reshape(n, QD)
            got = dev.download(out.ptr + ((i * L + l) * n * QD) * 2, (n, QD), np.uint16)
            for r in (0, n // 2, n - 1):
                T = t0 + r + 1
                t_cpu = time.perf_counter()
                ref = oracle_decode_layer(kvl[:, :T], T, ql[r], QH, D)
                cpu_s += time.perf_counter() - t_cpu
                cpu_pairs += T
                err = np.abs(got[r].view(np.float16).astype(np.float32) - ref)
                worst = max(worst, float(err.max()))
                ok = ok and bool(np.all(err <= 2e-3 + 1e-3 * np.abs(ref)))
                rows += 1
    cpu_tflops = 4.0 * QH * D * cpu_pairs / cpu_s / 1e12
    cpu = {"value": round(cpu_tflops, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
           "us_per_launch_equivalent": round(flops / (cpu_tflops * 1e12) * 1e6, 1),
           "sample": f"the check's {rows} query rows (one token's GQA decode over its {cpu_pairs // rows}-token mean "
                     f"causal context each, page setup included) by the oracle's kvo_paged_decode on "
                     f"{host_cpu()['model']}, {round(cpu_s, 2)} s",
           "seconds": round(cpu_s, 2)}
    print(json.dumps({
        "metric": "chunked-prefill causal paged GQA attention (MFMA) TFLOP/s",
        "value": round(tflops, 2), "unit": "TFLOP/s", "higher_is_better": True,
        "prompt_tokens_per_s": round(lanes * n / (ms_per_step * 1e-3), 1),
        "ms_per_step": round(ms_per_step, 3), "us_per_layer": round(ms_per_step * 1000.0 / L, 2),
        "prefill_kernel_avg_us": round(kernel_ms * 1000, 2), "prefill_launches": pf_n,
        "dtype": "f16 in, f32 accumulate",
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_MFMA_F16_TFLOPS, 4),
                     "traffic": profiled_traffic("prefill_kernel_chunked.md", chunks=lanes, chunk_tokens=n,
                                                 context_tokens=int(sum(int(t) for t in T0)), layers=L),
                     "kernel": "prefill_kernel", "launch_ms": round(kernel_ms, 4), "timed_launches": pf_n,
                     "flops_per_launch": flops,
                     "kv_q_o_bytes_per_launch": kv_bytes,
                     "hbm_gb_per_s_if_read_once": round(kv_bytes / (kernel_ms * 1e-3) / 1e9, 1)},
        "config": {"workload": f"{lanes} x {n}-token prefill chunks on contexts "
                               f"{'U[256, 2048]' if not args.prefill_context else 'of'} "
                               f"({', '.join(str(int(t)) for t in T0)}), {L} layers TinyLlama GQA 32q/4kv/64d fp16, "
                               f"forked per step (partial-tail COW), through the engine"},
        "steps": args.steps, "warmup": args.warmup,
        "check": {"rows": rows, "layers": [0, L - 1], "max_abs_err": worst, "within_tolerance": ok,
                  "tolerance": "2e-3 + 1e-3*|ref|"},
        "cpu_baseline": cpu_on_host(cpu)}), flush=True)
    return 0 if ok else 1


def run_e2e(kimkv, dev, args) -> int:
    """End-to-end TinyLlama-1.1B-shaped fp16 model (seeded N(0, 0.02) weights,
    RMSNorm weights one) under the iteration scheduler, in the steady state of
    --e2e-prefill requests doing --prefill-chunk-token chunked prefill (prompts
    U[256, 2048]) beside --e2e-decode decode lanes.  Setup (untimed): the
    decode lanes (prompts U[256, 1536], enough new tokens to outlive the run)
    are prefilled until every one is decoding.  Each timed step is one
    scheduler iteration under a budget of prefill * chunk + decode positions:
    one model call with every decode lane's next token and each prefilling
    request's next chunk; a prefilling request asks for one new token, so it
    leaves when its prompt completes and is replaced, keeping the mix fixed.
    Check: a short request through the same scheduler, teacher-forced through
    the oracle's CPU forward of the same model (every GPU token within 0.035
    of the oracle's max logit)."""
    import importlib
    host = importlib.import_module(kimkv.__name__ + ".host")
    L, KVH, D, QH, HID, INTER, VOC, MAXPOS = 22, 4, 64, 32, 2048, 5632, 32000, 2048
    n_dec, n_pre, chunk = args.e2e_decode, args.e2e_prefill, args.prefill_chunk
    budget = n_pre * chunk + n_dec
    rng = np.random.default_rng(args.seed)
    micro_cap = (n_dec * 2048 + (2 * n_pre + 2) * 2048) // 8 + 256
    engine = host.Engine(L, KVH, D, QH, 1 << 20, micro_cap, 16)
    assert engine.permute_free_slots(0, args.seed) == 0
    stream = dev.Stream()
    model = host.ModelConfig(HID, INTER, L, QH, KVH, D, VOC, MAXPOS, 1, 2, 1e-5, 10000.0)
    t0 = time.time()
    runner = host.Runner(engine, model, args.seed, budget + 64, n_dec + n_pre + 8, stream)
    sched = host.Scheduler(engine, runner, max_active=n_dec + n_pre + 8, max_batched_tokens=budget,
                           max_kv_tokens=1 << 40, prefill_chunk=chunk)
    log(f"model ready ({runner.weight_bytes() / 2**30:.2f} GiB of weights) in {time.time() - t0:.1f}s")
    next_id = [1]

    def submit(lo, hi, max_new):
        rid = next_id[0]
        next_id[0] += 1
        n = int(rng.integers(lo, hi + 1))
        assert sched.submit(rid, rng.integers(3, VOC, n), max_new) == "none"
        return rid

    decoders = [submit(256, 1536, 400) for _ in range(n_dec)]
    t0 = time.time()
    setup_iters = 0
    while True:
        r = sched.run_iteration()
        setup_iters += 1
        if r.prefill_tokens == 0:
            break
    finished = sched.take_terminals()
    assert not finished, finished[:1]
    log(f"{n_dec} decode lanes prefilled in {setup_iters} iterations ({time.time() - t0:.1f}s)")
    prefilling = set()

    def step():
        while len(prefilling) < n_pre:
            prefilling.add(submit(256, 2048, 1))
        r = sched.run_iteration()
        for t in sched.take_terminals():
            assert t["error"] == "none", t
            prefilling.discard(t["request_id"])
        return r

    for _ in range(args.warmup):
        step()
    # Events bracket every 5th attention launch (22 per step of each kind),
    # so the timing costs the iteration little.
    dev.prefill_timing(True, every=5)
    dev.decode_timing(True, every=5)
    tok_pre = tok_dec = 0
    t_wall = time.perf_counter()
    for _ in range(args.steps):
        r = step()
        tok_pre += r.prefill_tokens
        tok_dec += r.decode_tokens
    wall = time.perf_counter() - t_wall
    pf_ms, pf_n = dev.prefill_timing(False)
    dc_ms, dc_n = dev.decode_timing(False)
    ms_per_step = wall * 1000.0 / args.steps

    # Correctness sample: a short request through the same scheduler.
    import oracle.model as om
    prompt = [int(t) for t in rng.integers(3, VOC, 6)]
    rid = next_id[0]
    assert sched.submit(rid, prompt, 3) == "none"
    out = []
    for _ in range(64):
        sched.run_iteration()
        got = [t for t in sched.take_terminals() if t["request_id"] == rid]
        if got:
            out = got[0]["tokens"]
            break
    t0 = time.time()
    ref = om.ReferenceModel(om.ModelConfig(HID, INTER, L, QH, KVH, D, VOC, MAXPOS), args.seed)
    # The oracle's token-by-token forwards are also the CPU baseline.
    fwd_s, fwd_n = 0.0, 0

    def forward(tok, pos):
        nonlocal fwd_s, fwd_n
        t = time.perf_counter()
        r = ref.forward(tok, pos)
        fwd_s += time.perf_counter() - t
        fwd_n += 1
        return r

    for p, t in enumerate(prompt):
        logits = forward(t, p)
    ok, margin = len(out) == 3, 0.0
    for g, tok in enumerate(out):
        margin = max(margin, float(logits.max() - logits[tok]))
        ok = ok and bool(logits[tok] >= logits.max() - 0.035)
        if g + 1 < len(out):
            logits = forward(tok, len(prompt) + g)
    log(f"oracle check in {time.time() - t0:.1f}s")
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max((int(i.get("num_threads", 1)) for i in threadpool_info()), default=1)
    except ImportError:
        blas_threads = 1
    cpu = {"value": round(fwd_n / fwd_s, 2) if fwd_s > 0 else None, "unit": "tokens/s", "cores": blas_threads,
           "kind": "port",
           "sample": f"the check's {fwd_n} single-token forwards (positions 0-{fwd_n - 1}) through the oracle's "
                     f"fp32/fp16-rounded numpy model of the same weights on "
                     f"{host_cpu()['model']}, {round(fwd_s, 2)} s; no batching",
           "seconds": round(fwd_s, 2)}
    sched.close()
    runner.close()
    total = tok_pre + tok_dec
    per_layer_weights = HID * (QH * D + 2 * KVH * D) + QH * D * HID + HID * 2 * INTER + INTER * HID
    lin_flops = 2.0 * L * per_layer_weights * total
    print(json.dumps({
        "metric": "e2e TinyLlama chunked prefill + decode tokens/s (iteration scheduler)",
        "value": round(total / wall, 1), "unit": "tokens/s", "higher_is_better": True,
        "decode_tokens_per_s": round(tok_dec / wall, 1), "prefill_tokens_per_s": round(tok_pre / wall, 1),
        "ms_per_step": round(ms_per_step, 3), "tokens_per_step": round(total / args.steps, 1),
        "attention_ms_per_step": {"prefill_kernel": round(pf_ms / max(pf_n, 1) * L, 3),
                                  "decode_kernel": round(dc_ms / max(dc_n, 1) * L, 3),
                                  "timed_launches": [pf_n, dc_n]},
        "dtype": "f16 in, f32 accumulate",
        "config": {"workload": f"TinyLlama-1.1B-shaped fp16 (22 layers, hidden 2048, SwiGLU 5632, 32q/4kv x 64, "
                               f"vocab 32000), seeded N(0, 0.02) weights; {n_pre} requests in {chunk}-token chunked "
                               f"prefill (prompts U[256, 2048]) + {n_dec} decode lanes per iteration, greedy",
                   "max_batched_tokens": budget},
        "steps": args.steps, "warmup": args.warmup, "data": "synthetic (random token ids, seeded weights)",
        "check": {"request_prompt": 6, "tokens": len(out), "all_near_argmax": ok,
                  "max_logit_gap_to_oracle_max": margin, "tolerance": 0.035},
        "roofline": {"bound": "mfma", "achieved": round(lin_flops / wall / 1e12, 2), "peak": PEAK_MFMA_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(lin_flops / wall / 1e12 / PEAK_MFMA_F16_TFLOPS, 4),
                     "traffic": None, "kernel": "whole iteration",
                     "flops_per_step": round(lin_flops / args.steps),
                     "note": "FLOPs of the 22 layers' four linear projections (2 x 968.9 M weights per token) "
                             "over the step's wall time; attention and the LM head are not counted"},
        "cpu_baseline": cpu_on_host(cpu)}), flush=True)
    return 0 if ok else 1


def run_copy(dev, args) -> int:
    """Plain device-to-device copy of a known size: the achievable copy
    bandwidth of the box and the calibration run for the FETCH_SIZE /
    WRITE_SIZE counters."""
    nbytes = args.copy_mib << 20
    src, dst = dev.DeviceBuffer(nbytes), dev.DeviceBuffer(nbytes)
    dev.fill_rows(src.ptr, nbytes // 2, args.seed, 0, 4096)
    stream = dev.Stream()
    lib = dev.lib()
    sh = ctypes.c_void_p(stream.handle)
    for _ in range(args.warmup):
        dev.check(lib.kimkv_memcpy_d2d_async(ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), nbytes, sh), "copy")
    stream.synchronize()
    start, stop = dev.Event(), dev.Event()
    start.record(stream)
    for _ in range(args.steps):
        dev.check(lib.kimkv_memcpy_d2d_async(ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), nbytes, sh), "copy")
    stop.record(stream)
    stop.synchronize()
    ms = start.elapsed_ms(stop) / args.steps
    moved = 2 * nbytes
    print(json.dumps({"metric": "device-to-device copy GB/s (read + write)",
                      "value": round(moved / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
                      "us_per_copy": round(ms * 1000, 2), "read_bytes": nbytes, "write_bytes": nbytes,
                      "pct_of_peak_hbm": round(100 * moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
                      "steps": args.steps}), flush=True)
    return 0


def profiled_traffic(profile: str, **shape):
    """HBM bytes per launch from a committed rocprofv3 PMC summary under
    profiles/ (FETCH_SIZE and WRITE_SIZE per dispatch, each times its
    copy-calibrated factor), when the summary's machine-readable lines name
    the same workload shape as `shape`; None otherwise."""
    path = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(path):
        return None
    vals = {}
    block = False
    for line in open(path):
        block = block or line.startswith("Machine-readable")
        if block and ":" in line:
            k, _, v = line.strip().partition(":")
            try:
                vals[k.strip()] = float(v)
            except ValueError:
                pass
    try:
        if any(vals[k] != float(v) for k, v in shape.items()):
            return None
        return int(vals["fetch_size_kib_per_dispatch"] * 1024 * vals["fetch_factor"]
                   + vals["write_size_kib_per_dispatch"] * 1024 * vals["write_factor"])
    except KeyError:
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", choices=["decode", "parity", "gather", "append", "shared", "prefill", "e2e", "copy"],
                    default="decode",
                    help="decode: HBM-scale decode+append (the headline line); gather: long-sequence gather; "
                         "append: ragged one-token append with tail allocation; shared: fork/COW shared-prefix "
                         "decode; prefill: chunked-prefill attention through the engine; e2e: TinyLlama under the iteration "
                         "scheduler; copy: plain device copy (bandwidth and counter calibration)")
    ap.add_argument("--append-lanes", type=int, default=64)
    ap.add_argument("--append-check", type=int, default=4, help="lanes gathered and compared bit-exactly")
    ap.add_argument("--path", choices=["engine", "kernel"], default="engine",
                    help="engine: EngineKvBackend token transactions (reserve / writeLayerBatch / attendLayerBatch / "
                         "commit); kernel: the C-ABI kernels driven directly with bench-built page tables")
    ap.add_argument("--group-streams", choices=["own", "shared"], default="own",
                    help="engine path: each lane group on its own stream (own) or all on one (shared)")
    ap.add_argument("--shared-groups", type=int, default=1,
                    help="shared config: lane groups (whole fork groups) pipelined on their own streams "
                         "(1 = the 32 lanes as one batch per step)")
    ap.add_argument("--groups", type=int, default=2,
                    help="engine path: lane groups pipelined against each other (1 = one batch per step)")
    ap.add_argument("--slots", choices=["permuted", "sequential"], default="permuted",
                    help="kernel path: page slots in seeded-permutation order (default) or in pool order")
    ap.add_argument("--prefill-lanes", type=int, default=4)
    ap.add_argument("--e2e-decode", type=int, default=60)
    ap.add_argument("--e2e-prefill", type=int, default=4)
    ap.add_argument("--prefill-chunk", type=int, default=512)
    ap.add_argument("--prefill-context", type=int, default=0,
                    help="prefill: the same context for every lane instead of U[256, 2048]")
    ap.add_argument("--copy-mib", type=int, default=4096)
    ap.add_argument("--gather-tokens", type=int, default=16384)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=16)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--lanes", type=int, default=256)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=22)
    ap.add_argument("--cpu-lanes", type=int, default=32, help="lanes in the CPU baseline sample (0 = skip)")
    ap.add_argument("--seed", type=int, default=20260829)
    ap.add_argument("--decode-mode", choices=["plan", "head_split", "guided"], default="plan",
                    help="kernel path: decode mode (default: the planner's choice)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}), flush=True)
        return 2

    kimkv = load_package()
    dev = kimkv.device
    if dev.device_count() == 0:
        print(json.dumps({"error": "no HIP device visible"}), flush=True)
        return 1
    if args.config == "parity":
        return run_parity(kimkv, dev, args)
    if args.config == "gather":
        return run_gather(dev, args)
    if args.config == "copy":
        return run_copy(dev, args)
    if args.config == "append":
        return run_append(kimkv, dev, args)
    if args.config == "shared":
        return run_shared(kimkv, dev, args)
    if args.config == "prefill":
        return run_prefill(kimkv, dev, args)
    if args.config == "e2e":
        return run_e2e(kimkv, dev, args)
    H, D, QH = 4, 64, 32
    total_steps = args.warmup + args.steps
    if args.path == "engine":
        w = EngineWorkload(kimkv, dev, args.lanes, args.context, args.layers, H, D, QH, total_steps, args.seed,
                           args.groups, group_streams=args.group_streams == "own")
        stream = w.stream
    else:
        w = Workload(dev, args.lanes, args.context, args.layers, H, D, QH, total_steps, args.seed,
                     permute=args.slots == "permuted")
        w.decode_mode = args.decode_mode
        stream = dev.Stream()

    for s in range(args.warmup):
        w.step(s, stream)
    if args.path == "engine":
        w.drain()
    stream.synchronize()
    log("warmup done")
    if args.path == "engine":
        w.reserve_s = w.commit_s = 0.0
        group_lanes = w.groups[0][0].n
        chunk, _, total = dev.decode_plan(w.engine.storage_handle(), [w.lane_tokens(args.warmup)] * group_lanes, QH)
        w.plan = (chunk, total)

    start, stop = dev.Event(), dev.Event()
    # Events bracket every 5th decode launch of the timed steps (5 is prime
    # to the 44 launches of a step, so the sample walks every layer and lane
    # group); events around every launch cost the stream ~1 % of a step.
    # With the lane groups on their own streams two launches overlap, and
    # every launch is timed so that the union of their intervals (the time
    # the decode kernel occupies the GPU) is known.
    multi = args.path == "engine" and len(w.streams) > 1
    dev.decode_timing(True, every=1 if multi else 5)
    dev.sync()
    t_wall = time.perf_counter()
    start.record(stream)
    for s in range(args.warmup, total_steps):
        w.step(s, stream)
    if args.path == "engine":
        w.drain()
    dev.sync()
    stop.record(stream)
    stop.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1000.0
    decode_ms_total, decode_launches = dev.decode_timing(False)
    decode_busy_ms = dev.decode_timing_busy()
    gpu_ms = start.elapsed_ms(stop)
    ms_per_step = max(gpu_ms, wall_ms) / args.steps

    # Algorithmic bytes of the timed steps.
    tok_bytes = 2 * H * D * 2
    qo_bytes = 2 * QH * D * 2
    decode_bytes = 0
    append_bytes = 0
    for s in range(args.warmup, total_steps):
        T = w.lane_tokens(s)
        decode_bytes += args.layers * args.lanes * (T * tok_bytes + qo_bytes)
        append_bytes += args.layers * args.lanes * 2 * tok_bytes     # read new K/V + write page
    step_bytes = (decode_bytes + append_bytes) / args.steps
    value_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    lanes_per_launch = w.groups[0][0].n if args.path == "engine" else args.lanes
    # One decode launch per layer per lane group: bytes per launch (mean over
    # all timed launches) and time per launch (mean over the timed sample).
    launches = args.steps * args.layers * (len(w.groups) if args.path == "engine" else 1)
    # On the engine path a layer's decode launch also writes the lanes' new
    # tokens (kimkv_paged_decode_write_batch); the kernel path appends in a
    # launch of its own.
    fused_bytes = append_bytes if args.path == "engine" else 0
    per_launch_decode_bytes = (decode_bytes + fused_bytes) / launches
    decode_avg_ms = decode_ms_total / max(decode_launches, 1)
    # Per launch: its share of the time the decode kernel occupied the GPU.
    # One stream: the launches do not overlap and this is their mean
    # duration; several streams: the busy union over the launches.
    decode_eff_ms = decode_busy_ms / max(decode_launches, 1) if multi else decode_avg_ms
    achieved = per_launch_decode_bytes / (decode_eff_ms * 1e-3) / 1e9

    # Correctness sample + CPU baseline: lanes 0..k-1, layer 0, last step.
    last = total_steps - 1
    cpu = None
    check = None
    if args.cpu_lanes > 0:
        threads = max(1, min(16, os.cpu_count() or 1))
        outs, cpu_s, cpu_par_s, cpu_bytes = cpu_baseline(kimkv, w, args.cpu_lanes, last, threads)
        got = dev.download(w.out.ptr, (args.lanes, QH * D), np.uint16)   # layer 0 block
        errs = []
        for lane, ref in enumerate(outs):
            a = got[lane].view(np.float16).astype(np.float32)
            err = np.abs(a - ref)
            ok = bool(np.all(err <= 2e-3 + 1e-3 * np.abs(ref)))
            errs.append((float(err.max()), ok))
        check = {"lanes": args.cpu_lanes, "layer": 0, "max_abs_err": max(e for e, _ in errs),
                 "within_tolerance": all(ok for _, ok in errs), "tolerance": "2e-3 + 1e-3*|ref|"}
        cpu = {"value": round(cpu_bytes / cpu_s / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"oracle kvo_paged_decode, {args.cpu_lanes} lanes x 1 layer x {w.lane_tokens(last)} tokens "
                         f"(QH=32, H=4, D=64), {cpu_s:.1f}s on {host_cpu()['model']}",
               "seconds": round(cpu_s, 2),
               "all_cores": {"value": round(cpu_bytes / cpu_par_s / 1e9, 4), "unit": "GB/s", "cores": threads,
                             "seconds": round(cpu_par_s, 2),
                             "sample": f"the same {args.cpu_lanes} lane decodes over {threads} threads "
                                       f"(os.cpu_count() = {os.cpu_count()})"}}

    result = {
        "metric": "paged decode attn+append HBM GB/s (% peak) & us/layer, TinyLlama GQA, 1 GPU",
        "value": round(value_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "us_per_layer": round(ms_per_step * 1000.0 / args.layers, 1),
        "pct_of_peak_hbm": round(100.0 * value_gbs / PEAK_HBM_GBS, 1),
        "tokens_per_s": round(args.lanes / (ms_per_step * 1e-3), 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 storage, fp32 accumulate",
        "data": "synthetic (seeded Irwin-Hall fp16 K/V/Q generated on device)",
        "config": {"workload": f"HBM-scale decode: {args.lanes} lanes x {args.context}-token contexts "
                               f"(+{total_steps} appended), {args.layers} layers TinyLlama GQA 32q/4kv/64d fp16, "
                               f"extent pages in permuted slots, "
                               + ("through the engine token transactions" if args.path == "engine"
                                  else "kernels driven directly"),
                   "path": args.path,
                   "lanes": args.lanes, "context": args.context, "layers": args.layers,
                   "decode_mode": dev.decode_mode(w.plan[0]),
                   "decode_chunk_tokens": w.plan[0] & 0x3FFFFFFF if not w.plan[0] & dev.DECODE_GUIDED else None,
                   "decode_chunks_per_launch": w.plan[1],
                   "lane_groups": args.groups if args.path == "engine" else 1,
                   "group_streams": len(w.streams) if args.path == "engine" else 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("decode_kernel_hbm_scale.md", lanes_per_launch=lanes_per_launch,
                                                 context=args.context, layers=args.layers),
                     "kernel": "decode_kernel", "launch_ms": round(decode_eff_ms, 4),
                     "avg_launch_ms": round(decode_avg_ms, 4),
                     "launches_in_flight": round(decode_ms_total / decode_busy_ms, 3) if multi and decode_busy_ms
                     else 1.0,
                     "timed_launches": decode_launches, "launches": launches,
                     "lanes_per_launch": lanes_per_launch,
                     "bytes_per_launch": int(per_launch_decode_bytes)},
        "cpu_baseline": cpu_on_host(cpu),
        "check": check,
        "timing": {"gpu_event_ms": round(gpu_ms, 3), "wall_ms": round(wall_ms, 3)},
        "host": ({"path": "engine", "reserve_ms_per_step": round(w.reserve_s * 1000 / args.steps, 3),
                  "commit_ms_per_step": round(w.commit_s * 1000 / args.steps, 3)}
                 if args.path == "engine" else {"path": "kernel"}),
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
