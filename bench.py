"""Benchmark of the quantized data plane on one MI355X.

Headline (``value``): KV pack+unpack throughput in GB/s over the 7B-shaped
cache - 32 layers x B=1 x S=8192 x H=32 x D=128, bf16 K/V ~ N(0,1) with 1%
outlier channels x8, precision codes 25% fp16 / 50% int8 / 25% int4 (group
16) with a 4-token fp16 sink. One step = pack every layer (dense K/V ->
precision buckets), then unpack every layer (buckets -> fp32 K/V); inputs,
plans and buckets are resident in HBM before the timed region. A layer's
buckets are read back 31 launches after they were written and each K/V input
63 launches after its last read, with at least 6.5 GB of other traffic in
between (25x the 256 MB Infinity Cache plus the L2s), so every launch reads
its inputs from HBM; the steps run back to back between two synchronizations,
timed with HIP events on the launch stream.
Beside it: ``kv.flushed_*``, the same launches each preceded by an explicit
flush (a 512 MiB read, which leaves no dirty line behind) and timed alone
with an event pair, and ``kv.warm_*``, each unpack right after its own pack.
Throughput counts the algorithmic bytes: pack reads K+V and the code matrix
and writes the packed bytes; unpack reads the packed bytes and the codes and
writes fp32 K+V (slot metadata excluded).

Also reported on the same JSON line: per-kernel times with the roofline of the
dominant kernel, the INT8 FFN GEMM (4096 x 11008, M in {16, 64, 256, 1024}) in
TOPS against the int8 MFMA peak, the fused packed-KV attention, the
rate-distortion admission of one layer (sensitivity proxy + budget solver),
the paged KV store of one layer (prefill append, append, gather),
and the CPU baseline: the reference's own torch op chain on the host (a
bounded sample of the same workload, all cores of this job and 1 thread).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--part all|kv|gemm|attention|admit|paged|step|calib]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "shadow-infer_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, TOPS
FP16_PEAK_TFLOPS = 2500.0    # MI355X dense fp16/bf16 MFMA, TFLOP/s

LAYERS, B, S, H, D = 32, 1, 8192, 32, 128
GROUP = 16
CALIB_BYTES = 512 << 20
FLUSH_BYTES = 512 << 20      # > 256 MB Infinity Cache + 8 x 4 MB L2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_codes(seed: int):
    import numpy as np
    rng = np.random.default_rng(seed)
    codes = rng.choice(np.array([1, 2, 3], np.int8), size=(S, H), p=[0.25, 0.5, 0.25])
    codes[:4, :] = 1
    return codes


def make_kv(gen, device, dtype):
    import torch
    k = torch.randn(B, H, S, D, generator=gen, device=device)
    v = torch.randn(B, H, S, D, generator=gen, device=device)
    ch = torch.randperm(D, generator=gen, device=device)[: max(1, round(0.01 * D))]
    k[..., ch] *= 8
    v[..., ch] *= 8
    return k.to(dtype), v.to(dtype)


RAMP_MS = 60.0


def ramp(torch, fn, ms: float = RAMP_MS) -> None:
    """Run ``fn`` back to back, untimed, for at least ``ms`` milliseconds. The
    GPU raises its clocks over the first ~30 ms of sustained load after an
    idle gap (the packed attention at S=8192 runs 1384, 1227, 1186, then
    1177 us per launch in successive 10-launch windows), so every timed
    region below starts after such a ramp of its own launches."""
    t0 = time.perf_counter()
    batch = 1
    while True:
        for _ in range(batch):  # launches queue up back to back between synchronizations
            fn()
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= ms:
            return
        batch = min(2 * batch, 64)


class EventTimer:
    """HIP events recorded on the stream the kernels are launched on."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def time(self, fn, reps: int) -> float:
        torch = self.torch
        ramp(torch, fn)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(self.stream)
        for _ in range(reps):
            fn()
        end.record(self.stream)
        end.synchronize()
        return start.elapsed_time(end) / reps  # ms


def bench_kv(torch, dev, steps, warmup):
    from shadowinfer_amd import _native
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan

    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    gen = torch.Generator(device=dev).manual_seed(1234)
    layers = []
    for layer in range(LAYERS):
        k, v = make_kv(gen, dev, torch.bfloat16)
        codes = make_codes(1000 + layer)
        plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
        cache = PackedKVCache.pack(k, v, None, group_size=GROUP, plan=plan)["packed_kv"]
        code, slot, table, sdt, group = cache.device_state()
        ok = torch.empty(B, H, S, D, dtype=torch.float32, device=dev)
        ov = torch.empty_like(ok)
        flat = [plan.flat_indices[n] for n in ("fp32", "fp16", "int8", "int4")]
        counts = (ctypes.c_int64 * 5)(*plan.counts)
        # the raw pointer tables below stay valid while cache, plan and flat live in the dict
        layers.append(dict(k=k, v=v, code=code, slot=slot, table=table, sdt=sdt, cache=cache,
                           plan=plan, flat_lists=flat, ok=ok, ov=ov,
                           packed=cache.memory_bytes(), counts=counts,
                           flat=_native.table4([f.data_ptr() for f in flat])))
    torch.cuda.synchronize()

    def pack(L):
        _native.call("si_kv_pack_flat", L["k"].data_ptr(), L["v"].data_ptr(), _native.DT_BF16, B,
                     H, S, D, GROUP, L["code"].data_ptr(), L["slot"].data_ptr(), L["flat"],
                     L["counts"], L["table"], sptr)

    def unpack(L):
        _native.call("si_kv_unpack_flat", L["code"].data_ptr(), L["slot"].data_ptr(), L["flat"],
                     L["counts"], L["table"], L["sdt"], B, H, S, D, GROUP, L["ok"].data_ptr(),
                     L["ov"].data_ptr(), sptr)

    def step_warm():  # each unpack right after its own layer's pack
        for L in layers:
            pack(L)
            unpack(L)

    dense_in = 2 * B * H * S * D * 2          # K + V bf16
    codes_b = S * H                            # int8 codes
    fp32_out = 2 * B * H * S * D * 4           # K + V fp32
    pack_bytes = [dense_in + codes_b + L["packed"] for L in layers]
    unpack_bytes = [L["packed"] + codes_b + fp32_out for L in layers]
    step_bytes = sum(pack_bytes) + sum(unpack_bytes)
    avg_pack_b = sum(pack_bytes) / LAYERS
    avg_unpack_b = sum(unpack_bytes) / LAYERS

    # The headline: a step packs every layer, then unpacks every layer. A
    # layer's buckets are read back 31 launches after they were written, and
    # each K/V input 63 launches after its last read; between the two lie at
    # least 6.5 GB of other traffic, 25x the 256 MB Infinity Cache plus the
    # L2s, so no launch finds its inputs in a cache and every write-back of
    # the step is paid inside it. `steps` steps run back to back between two
    # synchronizations, timed by events on the launch stream; an event
    # between the pack and the unpack half of every step gives each kernel's
    # average launch time (32 launches per half, no event between them).
    def step_cold():
        for L in layers:
            pack(L)
        for L in layers:
            unpack(L)

    for _ in range(max(1, warmup)):
        step_cold()
    ramp(torch, step_cold)
    cev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    for r in range(steps):
        cev[r][0].record(stream)
        for L in layers:
            pack(L)
        cev[r][1].record(stream)
        for L in layers:
            unpack(L)
        cev[r][2].record(stream)
    torch.cuda.synchronize()
    c_wall = (time.perf_counter() - t0) / steps * 1e3
    c_step = cev[0][0].elapsed_time(cev[-1][2]) / steps
    c_pack = sum(e[0].elapsed_time(e[1]) for e in cev) / (steps * LAYERS)
    c_unpack = sum(e[1].elapsed_time(e[2]) for e in cev) / (steps * LAYERS)

    # The same step with each unpack right after its own pack (its buckets
    # partly still in the Infinity Cache): reported as warm_*.
    for _ in range(warmup):
        step_warm()
    torch.cuda.synchronize()
    timer = EventTimer(torch, stream)
    t0 = time.perf_counter()
    ms_step = timer.time(step_warm, steps)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3

    # Per-launch durations inside that warm loop: an event pair around every
    # pack and every unpack launch, on the launch stream.
    reps = max(2, steps // 4)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(LAYERS * reps)]
    for r in range(reps):
        for i, L in enumerate(layers):
            e0, e1, e2 = evs[r * LAYERS + i]
            e0.record(stream)
            pack(L)
            e1.record(stream)
            unpack(L)
            e2.record(stream)
    torch.cuda.synchronize()
    ms_pack = sum(e0.elapsed_time(e1) for e0, e1, _ in evs) / len(evs)
    ms_unpack = sum(e1.elapsed_time(e2) for _, e1, e2 in evs) / len(evs)

    # Explicit flushes: before every pack and every unpack launch a
    # FLUSH_BYTES buffer is read in full (a sum), which replaces the contents
    # of the Infinity Cache and of every L2 with clean lines, so each launch
    # reads its inputs from HBM and no earlier write is still waiting to be
    # written back (a flush by overwriting would leave that write-back to the
    # timed launch); each launch is timed alone with an event pair, which
    # adds its dispatch gap. Reported as flushed_*.
    flush_buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)

    def flush():
        flush_buf.sum(dtype=torch.int64)

    for L in layers[:2]:
        flush()
        pack(L)
        flush()
        unpack(L)
    fev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(LAYERS * steps)]
    torch.cuda.synchronize()
    for r in range(steps):
        for i, L in enumerate(layers):
            e = fev[r * LAYERS + i]
            flush()
            e[0].record(stream)
            pack(L)
            e[1].record(stream)
            flush()
            e[2].record(stream)
            unpack(L)
            e[3].record(stream)
    torch.cuda.synchronize()
    f_pack = [e[0].elapsed_time(e[1]) for e in fev]
    f_unpack = [e[2].elapsed_time(e[3]) for e in fev]
    f_step_ms = (sum(f_pack) + sum(f_unpack)) / steps
    fp = sum(f_pack) / len(f_pack)
    fu = sum(f_unpack) / len(f_unpack)
    del flush_buf
    res = {
        "protocol": "each step packs all 32 layers, then unpacks them: a layer's buckets are "
                    "read back 31 launches (>= 6.5 GB of traffic) after they were written, every "
                    "K/V input 63 launches after its last read; steps timed back to back",
        "ms_per_step": c_step,
        "wall_ms_per_step": c_wall,
        "step_bytes": step_bytes,
        "gbs": step_bytes / (c_step * 1e-3) / 1e9,
        "pack_us": c_pack * 1e3,
        "unpack_us": c_unpack * 1e3,
        "pack_gbs": avg_pack_b / (c_pack * 1e-3) / 1e9,
        "unpack_gbs": avg_unpack_b / (c_unpack * 1e-3) / 1e9,
        "pack_bytes_per_launch": avg_pack_b,
        "unpack_bytes_per_launch": avg_unpack_b,
        "packed_bytes_per_layer": sum(L["packed"] for L in layers) / LAYERS,
        # explicit 512 MiB flush read before every launch, each launch timed alone
        "flushed_ms_per_step": f_step_ms,
        "flushed_gbs": step_bytes / (f_step_ms * 1e-3) / 1e9,
        "flushed_pack_us": fp * 1e3,
        "flushed_unpack_us": fu * 1e3,
        "flushed_pack_gbs": avg_pack_b / (fp * 1e-3) / 1e9,
        "flushed_unpack_gbs": avg_unpack_b / (fu * 1e-3) / 1e9,
        # back to back, each unpack right after its own layer's pack
        "warm_ms_per_step": ms_step,
        "warm_wall_ms_per_step": wall,
        "warm_gbs": step_bytes / (ms_step * 1e-3) / 1e9,
        "warm_pack_us": ms_pack * 1e3,
        "warm_unpack_us": ms_unpack * 1e3,
        "warm_pack_gbs": avg_pack_b / (ms_pack * 1e-3) / 1e9,
        "warm_unpack_gbs": avg_unpack_b / (ms_unpack * 1e-3) / 1e9,
    }

    # The reference-API path (plan given, buckets allocated per call, unpack
    # allocating its outputs), for context: one layer, wall clock.
    L0 = layers[0]
    plan0 = PrecisionPlan.from_codes(torch.from_numpy(make_codes(1000)).to(dev))

    def api_roundtrip():
        c = PackedKVCache.pack(L0["k"], L0["v"], None, group_size=GROUP, plan=plan0)["packed_kv"]
        c.unpack()

    for _ in range(3):
        api_roundtrip()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        api_roundtrip()
    torch.cuda.synchronize()
    res["api_layer_ms"] = (time.perf_counter() - t0) / 10 * 1e3

    # Plan build (from_codes on the device, including the host copy of the counts).
    codes_dev = torch.from_numpy(make_codes(1000)).to(dev)
    t0 = time.perf_counter()
    for _ in range(10):
        PrecisionPlan.from_codes(codes_dev)
    torch.cuda.synchronize()
    res["plan_from_codes_ms"] = (time.perf_counter() - t0) / 10 * 1e3

    # Fused compression (working copy + buckets in one pass, 50% of the
    # entries reused from a previous K/V) on one layer.
    Lc, Lp = layers[0], layers[1]
    wk = torch.empty_like(Lc["k"])
    wv = torch.empty_like(Lc["v"])
    reuse_u8 = (torch.rand(S * H, generator=gen, device=dev) < 0.5).to(torch.uint8)

    def compress():
        _native.call("si_kv_pack_copy", Lc["k"].data_ptr(), Lc["v"].data_ptr(), _native.DT_BF16,
                     B, H, S, D, GROUP, Lc["code"].data_ptr(), Lc["slot"].data_ptr(), Lc["table"],
                     Lp["k"].data_ptr(), Lp["v"].data_ptr(), reuse_u8.data_ptr(), wk.data_ptr(),
                     wv.data_ptr(), sptr)

    compress()
    ms_c = timer.time(compress, 10)
    n_reuse = int(reuse_u8.sum().item())
    c_bytes = (dense_in + codes_b + S * H + Lc["packed"] + dense_in
               + n_reuse * B * D * 2 * 2)  # + previous rows of the reused entries
    res["compress_us"] = ms_c * 1e3
    res["compress_gbs"] = c_bytes / (ms_c * 1e-3) / 1e9
    res["compress_bytes"] = c_bytes

    # apply_reuse_mask (50% of the token-heads, previous step's cache packed
    # with the same plan) and evict (25%) on one layer, timed at the ABI like
    # pack/unpack. Algorithmic bytes: every reused entry is read from the
    # previous buckets and written into the current ones; evict reads and
    # writes every surviving entry of the buckets it rebuilds.
    L0 = layers[0]
    k2, v2 = make_kv(gen, dev, torch.bfloat16)
    prev = PackedKVCache.pack(k2, v2, None, group_size=GROUP, plan=L0["plan"])["packed_kv"]
    pcode, pslot, ptable, _, _ = prev.device_state()
    cur = L0["cache"]
    entry_b = torch.tensor([2 * B * D * 4, 2 * B * D * 2, 2 * B * (D + 2), 2 * B * (D // 2 + 2 * (D // GROUP)), 0],
                           dtype=torch.int64, device=dev)  # K + V bytes of one token-head per code
    code_l = L0["code"].to(torch.int64)
    reuse_m = (torch.rand(S * H, generator=gen, device=dev) < 0.5)
    reuse_u8m = reuse_m.to(torch.uint8)

    def reuse():
        _native.call("si_kv_reuse_flat", L0["flat"], L0["counts"], L0["table"], S, pcode.data_ptr(),
                     pslot.data_ptr(), ptable, S, reuse_u8m.data_ptr(), H, B, D, GROUP, L0["sdt"],
                     None, sptr)

    reuse()
    ms_reuse = timer.time(reuse, 20)
    r_bytes = int((entry_b[code_l] * reuse_m).sum()) * 2 + S * H * 11  # + codes, slots, mask
    res["reuse50_us"] = ms_reuse * 1e3
    res["reuse50_bytes"] = r_bytes
    res["reuse50_gbs"] = r_bytes / (ms_reuse * 1e-3) / 1e9
    t0 = time.perf_counter()
    for _ in range(5):
        cur.apply_reuse_mask(prev, reuse_m.view(S, H))
    torch.cuda.synchronize()
    res["reuse50_api_us"] = (time.perf_counter() - t0) / 5 * 1e6

    ev_m = (torch.rand(S * H, generator=gen, device=dev) < 0.25)
    ev_u8 = ev_m.to(torch.uint8)
    # PackedKVCache.evict: pass 1 over the old lists (new codes, chunk survivor
    # counts), the host reads the new sizes from the chunk counts, pass 2
    # compacts. The timed region holds the two device passes.
    grp = L0["plan"].device_grouping()
    o_flat_t = _native.table4([f.data_ptr() for f in grp.flat_lists(S, H)])
    o_cnt = (ctypes.c_int64 * 4)(*[int(c) for c in grp.counts[:4]])
    chunks = int(_native.load().si_kv_evict_chunks(o_cnt))
    cc = torch.empty(max(chunks, 1), dtype=torch.int32, device=dev)
    bits = torch.empty(max(chunks * int(_native.load().si_kv_evict_chunk_words()), 1),
                       dtype=torch.int64, device=dev)
    n_code = torch.empty(S * H, dtype=torch.int8, device=dev)
    n_slot = torch.empty(S * H, dtype=torch.int32, device=dev)
    new_counts = grp.evict_count(ev_u8, S, H)[3]
    fresh = cur._alloc_buckets(new_counts, dev, torch.bfloat16)
    ftable = cur._bucket_table(fresh)
    n_flat = [torch.empty(c, dtype=torch.long, device=dev) for c in new_counts[:4]]
    n_flat_t = _native.table4([f.data_ptr() for f in n_flat])
    n_counts = (ctypes.c_int64 * 4)(*new_counts[:4])

    def evict():  # the device work of PackedKVCache.evict: count pass, compaction pass
        _native.call("si_kv_evict_count", L0["code"].data_ptr(), o_flat_t, o_cnt, ev_u8.data_ptr(),
                     S, H, n_code.data_ptr(), n_slot.data_ptr(), cc.data_ptr(), bits.data_ptr(), sptr)
        _native.call("si_kv_evict_flat", o_flat_t, o_cnt, cc.data_ptr(), bits.data_ptr(), S, H,
                     L0["table"], n_flat_t, n_counts, ftable, n_slot.data_ptr(), B, D, GROUP,
                     L0["sdt"], sptr)

    evict()
    ms_ev = timer.time(evict, 20)
    kept = ~ev_m & (code_l < 4)
    e_bytes = int((entry_b[code_l] * kept).sum()) * 2 + S * H * 16  # + codes, slots, mask
    res["evict25_us"] = ms_ev * 1e3
    res["evict25_bytes"] = e_bytes
    res["evict25_gbs"] = e_bytes / (ms_ev * 1e-3) / 1e9
    times = []
    for _ in range(3):  # the first call is a warm-up
        victim = PackedKVCache.pack(k2, v2, None, group_size=GROUP, plan=L0["plan"])["packed_kv"]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        victim.evict(ev_m.view(S, H))
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    res["evict25_api_us"] = min(times[1:]) * 1e6
    # The reference's own input forms (packed_kv_cache.py:666-854): a Python
    # set of (token, head) pairs for evict, a dict for apply_reuse_mask; the
    # wall clock includes turning them into the device mask.
    import numpy as np
    ev_pairs = np.argwhere(ev_m.view(S, H).cpu().numpy())
    ev_set = set(zip(ev_pairs[:, 0].tolist(), ev_pairs[:, 1].tolist()))
    ru_pairs = np.argwhere(reuse_m.view(S, H).cpu().numpy())
    ru_dict = {(int(t), int(h)): True for t, h in ru_pairs}
    cur.apply_reuse_mask(prev, ru_dict)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        cur.apply_reuse_mask(prev, ru_dict)
    torch.cuda.synchronize()
    res["reuse50_dict_api_ms"] = (time.perf_counter() - t0) / 3 * 1e3
    res["reuse50_dict_entries"] = len(ru_dict)
    times = []
    for _ in range(3):  # the first call is a warm-up
        victim = PackedKVCache.pack(k2, v2, None, group_size=GROUP, plan=L0["plan"])["packed_kv"]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        victim.evict(ev_set)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    res["evict25_set_api_ms"] = min(times[1:]) * 1e3
    res["evict25_set_entries"] = len(ev_set)
    # The freed layers stay in torch's caching allocator for the parts that
    # follow, as in any long-running process. Handing them back to the driver
    # (torch.cuda.empty_cache) made the next part's fresh allocations land on
    # a remapped heap where the small-M GEMMs ran 5-20% slower (M=64 12.4 ->
    # 14.2-14.9 us): a property of that allocation history, not of the kernels.
    del layers
    return res


def bench_gemm(torch, dev, iters=50):
    from shadowinfer_amd import _native

    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    K, N = 4096, 11008
    gen = torch.Generator(device=dev).manual_seed(7)
    copies = 8  # 8 x 45 MB of weights: more than the 256 MB last-level cache
    # W ~ N(0, 0.02) quantized per output channel (INT8Linear.from_linear's
    # arithmetic, si_weight_quant_i8), kept in nn.Linear's [N, K] layout.
    ws = []
    sw = torch.empty(N, dtype=torch.float32, device=dev)
    for _ in range(copies):
        w = torch.randn(N, K, generator=gen, device=dev) * 0.02
        q = torch.empty(N, K, dtype=torch.int8, device=dev)
        _native.call("si_weight_quant_i8", w.data_ptr(), N, K, q.data_ptr(), sw.data_ptr(), sptr)
        ws.append(q)
        del w
    timer = EventTimer(torch, stream)
    out = {}
    for M in (16, 64, 256, 1024):
        x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        q = torch.empty(M, K, dtype=torch.int8, device=dev)
        sx = torch.empty(M, dtype=torch.float32, device=dev)
        c = torch.empty(M, N, dtype=torch.int32, device=dev)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        gws_b = _native.size_query("si_gemm_workspace_bytes", M, N, K)
        gws = torch.empty(max(gws_b, 1), dtype=torch.uint8, device=dev)
        lws_b = _native.size_query("si_int8_linear_workspace_bytes", M, K, N)
        lws = torch.empty(lws_b, dtype=torch.uint8, device=dev)
        _native.call("si_act_quant_i8", x.data_ptr(), _native.DT_BF16, M, K, q.data_ptr(),
                     sx.data_ptr(), sptr)
        it = [0]
        # The library entry points are bound once and their arguments built
        # before the timed loops: at 10-15 us per launch, Python-side argument
        # marshalling per call would otherwise set the pace instead of the GPU.
        lib = _native.load()
        f_gemm, f_fwd, f_deq = lib.si_gemm_i8i8_i32, lib.si_int8_linear_forward, lib.si_gemm_i8_dequant
        a_gemm = [(q.data_ptr(), w.data_ptr(), M, N, K, c.data_ptr(), gws.data_ptr(), gws_b, sptr)
                  for w in ws]
        a_fwd = [(x.data_ptr(), _native.DT_BF16, M, K, N, w.data_ptr(), sw.data_ptr(), None,
                  y.data_ptr(), lws.data_ptr(), lws_b, sptr) for w in ws]
        a_deq = [(q.data_ptr(), sx.data_ptr(), w.data_ptr(), sw.data_ptr(), None, M, N, K,
                  y.data_ptr(), _native.DT_BF16, gws.data_ptr(), gws_b, sptr) for w in ws]
        rcs = []

        def gemm():
            i = it[0] % copies
            it[0] += 1
            rcs.append(f_gemm(*a_gemm[i]))

        def forward():
            i = it[0] % copies
            it[0] += 1
            rcs.append(f_fwd(*a_fwd[i]))

        def gemm_dequant():  # the GEMM with INT8Linear's epilogue, bf16 out
            i = it[0] % copies
            it[0] += 1
            rcs.append(f_deq(*a_deq[i]))

        for _ in range(5):
            gemm()
            forward()
            gemm_dequant()
        ms_gemm = timer.time(gemm, iters)
        ms_deq = timer.time(gemm_dequant, iters)
        ms_fwd = timer.time(forward, iters)
        if any(rc != 0 for rc in rcs):
            raise RuntimeError(f"INT8 GEMM launch failed: {lib.si_last_error().decode(errors='replace')}")
        ops = 2.0 * M * K * N
        # The vendor library on the same operands: hipBLASLt through
        # torch._int_mm (it needs more than 16 rows), weight as the [K, N]
        # view of the [N, K] buffers, int32 out.
        vendor = None
        if M > 16:
            def vendor_mm():
                w = ws[it[0] % copies]
                it[0] += 1
                torch._int_mm(q, w.t())
            for _ in range(3):
                vendor_mm()
            vendor = timer.time(vendor_mm, iters)
        out[str(M)] = {
            "gemm_us": ms_gemm * 1e3,
            "gemm_tops": ops / (ms_gemm * 1e-3) / 1e12,
            "gemm_frac": ops / (ms_gemm * 1e-3) / 1e12 / INT8_PEAK_TOPS,
            "gemm_weight_gbs": K * N / (ms_gemm * 1e-3) / 1e9,
            "gemm_dequant_us": ms_deq * 1e3,
            "gemm_dequant_frac": ops / (ms_deq * 1e-3) / 1e12 / INT8_PEAK_TOPS,
            "forward_us": ms_fwd * 1e3,
            "forward_tops": ops / (ms_fwd * 1e-3) / 1e12,
        }
        if vendor is not None:
            out[str(M)]["hipblaslt_int_mm_us"] = vendor * 1e3
            out[str(M)]["speedup_vs_hipblaslt"] = vendor / ms_gemm
    del ws
    return out


def bench_attention(torch, dev, iters=10):
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan, packed_attention

    res = {}
    gen = torch.Generator(device=dev).manual_seed(11)
    stream = torch.cuda.current_stream(dev)
    timer = EventTimer(torch, stream)
    for Sq in (2048, 8192):
        k = torch.randn(1, H, Sq, D, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(1, H, Sq, D, generator=gen, device=dev).to(torch.bfloat16)
        codes = torch.from_numpy(make_codes(5)[:Sq]).to(dev) if Sq <= S else None
        plan = PrecisionPlan.from_codes(codes)
        cache = PackedKVCache.pack(k, v, None, group_size=GROUP, plan=plan)["packed_kv"]
        q = torch.randn(1, H, Sq, D, generator=gen, device=dev).to(torch.bfloat16)
        for _ in range(2):
            packed_attention(q, cache)
        ms = timer.time(lambda: packed_attention(q, cache), iters)
        flops = 4.0 * H * Sq * Sq * D
        res[str(Sq)] = {"us": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12,
                        "frac": flops / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS}
    return res


def bench_admit(torch, dev, iters=20, with_cpu=True):
    """Admission for one layer (S=8192 x H=32 token-heads, B=1, D=128): the
    sensitivity proxy over bf16 K/V, then admit_codes from all-fp16 codes to a
    budget of half the bytes, and to a tenth with eviction."""
    import numpy as np
    from shadowinfer_amd.shadowkv import PrecisionPlan, admit_codes, kv_sensitivity

    stream = torch.cuda.current_stream(dev)
    timer = EventTimer(torch, stream)
    gen = torch.Generator(device=dev).manual_seed(77)
    k, v = make_kv(gen, dev, torch.bfloat16)
    res = {}
    kv_sensitivity(k, v)
    ms = timer.time(lambda: kv_sensitivity(k, v), iters)
    sens_bytes = 2 * k.numel() * 2 + S * H * 2
    res["sensitivity_us"] = ms * 1e3
    res["sensitivity_gbs"] = sens_bytes / (ms * 1e-3) / 1e9
    sens = kv_sensitivity(k, v).float()
    imp = torch.rand(S, H, generator=gen, device=dev)
    codes = torch.ones(S, H, dtype=torch.int8, device=dev)
    full = S * H * 2 * B * D * 2 * 2
    for name, budget, evict in (("half", full // 2, False), ("tenth_evict", full // 10, True)):
        admit_codes(codes, imp, sens, budget, B, D, sink_tokens=4, allow_eviction=evict)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            out, pred, ev = admit_codes(codes, imp, sens, budget, B, D, sink_tokens=4,
                                        allow_eviction=evict)
        res[f"admit_{name}_ms"] = (time.perf_counter() - t0) / iters * 1e3
        res[f"admit_{name}_predicted"] = pred
        res[f"admit_{name}_evicted"] = ev
    # sensitivity + admission + plan, as a caller runs them before a pack
    def plan_step():
        s_ = kv_sensitivity(k, v).float()
        out_, _, _ = admit_codes(codes, imp, s_, full // 2, B, D, sink_tokens=4)
        PrecisionPlan.from_codes(out_)
    plan_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        plan_step()
    torch.cuda.synchronize()
    res["sens_admit_plan_ms"] = (time.perf_counter() - t0) / iters * 1e3
    if with_cpu:
        sys.path.insert(0, ROOT)
        from oracle import oracle as O
        c_np, i_np, s_np = codes.cpu().numpy(), imp.cpu().numpy(), sens.cpu().numpy()
        t0 = time.perf_counter()
        for _ in range(3):
            O.admit_codes(c_np, i_np, s_np, full // 2, B, D, 4, True, False)
        res["cpu_admit_half_ms"] = (time.perf_counter() - t0) / 3 * 1e3
    return res


def bench_paged(torch, dev, iters=10):
    """PagedKVStore for one layer (B=1, H=32, D=128, bf16): an 8192-token
    int8 prefill into 32-token pages, a 64-token append, and gather (every
    page decoded to fp32 [1, 32, 8192, 128] in one launch)."""
    from shadowinfer_amd.shadowkv import PagedKVStore

    stream = torch.cuda.current_stream(dev)
    timer = EventTimer(torch, stream)
    gen = torch.Generator(device=dev).manual_seed(91)
    k, v = make_kv(gen, dev, torch.bfloat16)
    res = {}
    warm = PagedKVStore(B, H, D, page_size=32, device=dev)
    warm.append(k, v, "int8")  # first use: kernel load and allocator growth
    del warm
    st = PagedKVStore(B, H, D, page_size=32, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    st.append(k, v, "int8")
    torch.cuda.synchronize()
    res["prefill_append_ms"] = (time.perf_counter() - t0) * 1e3
    res["pages"] = st.page_count
    st.gather()
    ms = timer.time(st.gather, iters)
    payload = st.data_plane_bytes()
    out_bytes = 2 * B * H * S * D * 4
    res["gather_us"] = ms * 1e3
    res["gather_bytes"] = payload + out_bytes
    res["gather_gbs"] = (payload + out_bytes) / (ms * 1e-3) / 1e9
    st2 = PagedKVStore(B, H, D, page_size=32, device=dev)
    st2.append(k[:, :, :8128], v[:, :, :8128], "int8")
    kn, vn = k[:, :, 8128:].contiguous(), v[:, :, 8128:].contiguous()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    st2.append(kn, vn, "int8")
    torch.cuda.synchronize()
    res["append_64_tokens_us"] = (time.perf_counter() - t0) * 1e6
    return res


def bench_step(torch, dev, steps=8, warmup=2, gen_steps=64):
    """One denoising step of a random-init Llama-7B-shaped diffusion LM
    (32 layers, hidden 4096, 32 heads, SwiGLU 11008, vocab 32000) on B=1,
    S=2048 with 50% mask tokens: INT8 gate|up and down projections, per-layer
    packed KV rebuilt every step (codes 25% fp16 / 50% int8 / 25% int4 g16,
    4-token fp16 sink), step reuse on every other layer after the first step,
    one unmasking round per step. Reports the steady-state step (16 computed +
    16 reused layers), a step with every layer computed, and a whole
    64-step generation."""
    import numpy as np
    from shadowinfer_amd.execution import (DiffusionLlamaShape, PackedDiffusionLlama,
                                           StepReuseConfig, StepReuseState, mask_tokens)
    from shadowinfer_amd.shadowkv import PrecisionPlan

    cfg = DiffusionLlamaShape()
    Sd = 2048
    model = PackedDiffusionLlama(cfg, device=dev, seed=5)
    plans = []
    for i in range(cfg.num_hidden_layers):
        rng = np.random.default_rng(100 + i)
        codes = rng.choice(np.array([1, 2, 3], np.int8), size=(Sd, cfg.num_attention_heads),
                           p=[0.25, 0.5, 0.25])
        codes[:4, :] = 1
        plans.append(PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev)))
    # every other layer reused from the second step on, without the drift's
    # device read (skip_drift), so each step stays one asynchronous stream
    reuse_cfg = StepReuseConfig(enabled=True, threshold=float("inf"), warmup_steps=1,
                                reusable_layers=set(range(1, cfg.num_hidden_layers, 2)),
                                skip_drift=True)
    stream = torch.cuda.current_stream(dev)
    timer = EventTimer(torch, stream)
    res = {}

    def fresh():
        tokens, masked = mask_tokens(1, Sd, 0.5, cfg, dev, seed=7)
        return tokens, masked, StepReuseState()

    # every layer computed (no reuse state)
    tokens, masked, _ = fresh()
    for _ in range(warmup):
        model.forward_step(tokens, plans)
    res["full_step_ms"] = timer.time(lambda: model.forward_step(tokens, plans), steps)

    # steady state: step >= 1 with half the layers reused
    tokens, masked, state = fresh()
    model.denoise_step(tokens, masked, plans, 0, 0.9, state, reuse_cfg)
    it = iter(range(1, 10 ** 6))
    for _ in range(warmup):
        model.denoise_step(tokens, masked, plans, next(it), 0.9, state, reuse_cfg)
    res["step_ms"] = timer.time(
        lambda: model.denoise_step(tokens, masked, plans, next(it), 0.9, state, reuse_cfg), steps)
    res["reused_ratio"] = state.stats()["reused_ratio"]

    # a whole generation: step 0 computes every layer, then 63 reuse steps,
    # then the forced completion of what is still masked
    tokens, masked, state = fresh()
    n_masked = int(masked.sum())
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    gen = model.generate(tokens, masked, plans, gen_steps, 0.9, state, reuse_cfg)
    end.record(stream)
    end.synchronize()
    res["generation_ms"] = start.elapsed_time(end)
    res["generation_steps"] = gen_steps
    res["unmasked_in_rounds"] = int(gen["unmasked_per_step"].sum())
    res["forced_completions"] = int(gen["forced"].sum())
    res["masked_at_start"] = n_masked
    res["all_resolved"] = not bool(masked.any())
    res["positions_per_s"] = Sd / (res["step_ms"] * 1e-3)
    return res


def host_cpu():
    """CPU model name and CPU counts of the host this runs on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        import psutil
        physical = psutil.cpu_count(logical=False)
    except Exception:
        physical = None
    return {"cpu_model": model, "host_logical_cpus": os.cpu_count(),
            "host_physical_cores": physical, "affinity_cpus": len(os.sched_getaffinity(0))}


def all_threads() -> int:
    """Threads for the all-cores leg: this job's CPU share (OMP_NUM_THREADS
    when set, as on the GPU box), else the CPUs in the affinity mask, at most
    the physical cores."""
    info = host_cpu()
    n = info["affinity_cpus"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        n = min(n, int(os.environ["OMP_NUM_THREADS"]))
    if info["host_physical_cores"]:
        n = min(n, info["host_physical_cores"])
    return max(1, n)


def _stats(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2], xs[0], xs[-1]


def cpu_baseline(layers_all: int = 5, layers_one: int = 3):
    """The reference's CPU path for the headline workload: the torch op chain
    of PackedKVCache._do_pack_with_plan + unpack (oracle/torch_ref.py) on one
    7B layer at a time (each layer its own K/V and codes, the plan built
    beforehand as the reference's pack receives it), timed with perf_counter
    after a warm-up layer, once with torch.set_num_threads(all cores of this
    job) and once with 1 thread. GB/s over the same algorithmic bytes as the
    GPU line."""
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    from oracle import torch_ref as TR

    gen = torch.Generator().manual_seed(99)
    prev_threads = torch.get_num_threads()

    def layer_inputs(i):
        k = torch.randn(B, H, S, D, generator=gen)
        v = torch.randn(B, H, S, D, generator=gen)
        ch = torch.randperm(D, generator=gen)[: max(1, round(0.01 * D))]
        k[..., ch] *= 8
        v[..., ch] *= 8
        groups, flat = TR.plan_from_codes(torch.from_numpy(make_codes(1000 + i)))
        return k.to(torch.bfloat16), v.to(torch.bfloat16), groups, flat

    def run(threads, n):
        torch.set_num_threads(threads)
        rates, times = [], []
        for i in range(n + 1):
            k, v, groups, flat = layer_inputs(i)
            t0 = time.perf_counter()
            packed = TR.pack_with_plan(k, v, groups, flat, GROUP)
            TR.unpack(packed, B, H, S, D)
            dt = time.perf_counter() - t0
            pbytes = sum(t.numel() * t.element_size() for d in packed.values()
                         for key in ("k", "v", "scale_k", "scale_v")
                         for t in [d.get(key)] if t is not None)
            nbytes = (2 * B * H * S * D * 2 + S * H + pbytes) + (pbytes + S * H + 2 * B * H * S * D * 4)
            if i:                       # layer 0 warms up
                rates.append(nbytes / dt / 1e9)
                times.append(dt * 1e3)
        med, lo, hi = _stats(rates)
        return {"threads": threads, "layers": n, "median_gbs": med, "min_gbs": lo, "max_gbs": hi,
                "median_layer_ms": _stats(times)[0]}

    n_all = all_threads()
    t0 = time.perf_counter()
    res_all = run(n_all, layers_all)
    res_one = run(1, layers_one)
    torch.set_num_threads(prev_threads)
    return {"value": res_all["median_gbs"], "unit": "GB/s", "cores": n_all, "kind": "port",
            "sample": f"pack+unpack of one 7B layer at a time (1 x 32 x 8192 x 128 bf16, the "
                      f"headline's codes), the reference's torch op chain on the host: "
                      f"{layers_all} layers with {n_all} threads, {layers_one} with 1 thread, "
                      "median over layers after one warm-up layer",
            "threads_all": res_all, "threads_1": res_one, **host_cpu(),
            "seconds": time.perf_counter() - t0}


def cpu_gemm_baseline(ms=(16, 64, 256, 1024), reps_all=5, reps_one=3):
    """INT8Linear.forward's torch op chain with CPU torch._int_mm
    (oracle/torch_ref.py) on M x 4096 x 11008, bf16 input, weights N(0, 0.02)
    quantized per channel: median and range of ``reps`` calls after two
    warm-ups, with all cores of this job and with 1 thread."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import torch_ref as TR

    K, N = 4096, 11008
    gen = torch.Generator().manual_seed(5)
    qw, sw = TR.int8_weight(torch.randn(N, K, generator=gen) * 0.02)
    prev_threads = torch.get_num_threads()

    def run(threads, reps):
        torch.set_num_threads(threads)
        out = {"threads": threads}
        for M in ms:
            x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
            for _ in range(2):
                TR.int8_linear_forward(x, qw, sw)
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                TR.int8_linear_forward(x, qw, sw)
                ts.append(time.perf_counter() - t0)
            med, lo, hi = _stats(ts)
            out[str(M)] = {"ms": med * 1e3, "min_ms": lo * 1e3, "max_ms": hi * 1e3,
                           "tops": 2.0 * M * K * N / med / 1e12}
        return out

    n_all = all_threads()
    res = {"kind": "port", "cores": n_all,
           "sample": "INT8Linear forward torch op chain with CPU torch._int_mm, M x 4096 x 11008, "
                     f"median of {reps_all} ({n_all} threads) / {reps_one} (1 thread) calls",
           "threads_all": run(n_all, reps_all), "threads_1": run(1, reps_one), **host_cpu()}
    torch.set_num_threads(prev_threads)
    return res


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed counter summary
    (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by the factor a plain
    copy of known size gives); None when no summary is present."""
    path = os.path.join(ROOT, "profiles", "kv_7b_layer_hbm_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        pass
    return None


def _rounded(obj, nd=4):
    if isinstance(obj, float):
        return round(obj, nd)
    if isinstance(obj, dict):
        return {k: _rounded(v, nd) for k, v in obj.items()}
    return obj


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="same as --part kv")
    ap.add_argument("--part", choices=("all", "kv", "gemm", "attention", "admit", "paged",
                                       "step", "calib"),
                    default="all",
                    help="run one part only (for profiling); 'calib' runs the plain device "
                         "fill and copy that calibrate the HBM byte counters")
    args = ap.parse_args()
    if args.quick:
        args.part = "kv"
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    log(f"device {torch.cuda.get_device_name(dev)}")

    if args.part == "calib":
        # Counter calibration: a fill (writes CALIB_BYTES) and device-to-device
        # copies (read CALIB_BYTES, write CALIB_BYTES), nothing else.
        src = torch.empty(CALIB_BYTES, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "fill + 3 copies", "bytes": CALIB_BYTES}), flush=True)
        return
    if args.part in ("gemm", "attention", "admit", "paged", "step"):
        fn = {"gemm": bench_gemm, "attention": bench_attention, "admit": bench_admit,
              "paged": bench_paged, "step": bench_step}[args.part]
        log(args.part)
        print(json.dumps({args.part: fn(torch, dev)}), flush=True)
        return
    log("kv pack+unpack")
    kv = bench_kv(torch, dev, args.steps, args.warmup)
    log(f"kv {kv['gbs']:.1f} GB/s (pack {kv['pack_us']:.1f} us, unpack {kv['unpack_us']:.1f} us); "
        f"flushed per launch {kv['flushed_gbs']:.1f} GB/s; warm {kv['warm_gbs']:.1f} GB/s")
    gemm = attn = adm = paged = step = None
    if args.part == "all":
        log("int8 gemm")
        gemm = bench_gemm(torch, dev)
        log("attention")
        attn = bench_attention(torch, dev)
        log("admission")
        adm = bench_admit(torch, dev, with_cpu=not args.no_cpu)
        log("paged store")
        paged = bench_paged(torch, dev)
        log("denoising step")
        step = bench_step(torch, dev)
    cpu = None
    gemm_cpu = None
    if not args.no_cpu:
        log("cpu baseline (the reference's torch op chain on the host)")
        cpu = cpu_baseline()
        log(f"cpu {cpu['value']:.3f} GB/s ({cpu['cores']} threads), "
            f"{cpu['threads_1']['median_gbs']:.3f} GB/s (1 thread) in {cpu['seconds']:.1f} s")
        if gemm is not None:
            gemm_cpu = cpu_gemm_baseline()
            log("cpu gemm " + ", ".join(f"M={m} {gemm_cpu['threads_all'][m]['ms']:.2f} ms"
                                         for m in ("16", "64", "256", "1024")))

    dom = "unpack" if kv["unpack_us"] >= kv["pack_us"] else "pack"
    achieved = kv[f"{dom}_gbs"]
    line = {
        "metric": "KV pack+unpack GB/s (%HBM peak); INT8 FFN GEMM TOPS (%MFMA peak)",
        "value": round(kv["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kv["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "PackedKVCache pack+unpack, 32 layers x B=1 x S=8192 x H=32 x D=128, "
                        "bf16 K/V, codes 25% fp16 / 50% int8 / 25% int4 g16, 4-token fp16 sink",
            "layers": LAYERS, "batch": B, "seq_len": S, "heads": H, "head_dim": D,
            "int4_group": GROUP, "hbm_frac": round(kv["gbs"] / HBM_PEAK_GBS, 4),
            "protocol": "pack all 32 layers, then unpack them; each launch's inputs last "
                        "touched >= 6.5 GB of traffic earlier (cold); steps timed back to back",
        },
        "roofline": {
            "kernel": f"kv_{dom}",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(f"kv_{dom}"),
            "traffic_source": "profiles/kv_7b_layer_hbm_traffic.txt: rocprofv3 --pmc FETCH_SIZE "
                              "and WRITE_SIZE per dispatch of this bench's kv part, each scaled "
                              "by the counter's reading for a plain device copy",
            "bytes_per_launch": int(kv[f"{dom}_bytes_per_launch"]),
            "avg_launch_us": round(kv[f"{dom}_us"], 3),
        },
        "cpu_baseline": cpu and _rounded({k: v for k, v in cpu.items() if k != "seconds"}),
        "kv": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in kv.items()},
    }
    if gemm is not None:
        line["int8_gemm"] = {"shape": "M x 4096 x 11008", "peak_tops": INT8_PEAK_TOPS,
                             **{m: {k: round(v, 4) for k, v in r.items()} for m, r in gemm.items()}}
        if gemm_cpu is not None:
            line["int8_gemm"]["cpu_baseline"] = _rounded(gemm_cpu)
    if attn is not None:
        line["packed_attention"] = {"shape": "B=1, H=32, D=128, S_q=S_kv", "peak_tflops": FP16_PEAK_TFLOPS,
                                    **{s: {k: round(v, 4) for k, v in r.items()} for s, r in attn.items()}}
    if paged is not None:
        line["paged_kv_store"] = {"shape": "B=1, H=32, D=128, bf16 K/V, int8 pages of 32 tokens",
                                  **{k: (round(v, 4) if isinstance(v, float) else v)
                                     for k, v in paged.items()}}
    if adm is not None:
        line["admission"] = {"shape": "S=8192 x H=32 token-heads, B=1, D=128, bf16 K/V",
                             **{k: (round(v, 4) if isinstance(v, float) else v)
                                for k, v in adm.items()}}
    if step is not None:
        line["denoising_step"] = {
            "shape": "Llama-7B-shaped diffusion LM, 32 layers, hidden 4096, 32 heads, SwiGLU 11008, "
                     "vocab 32000, B=1, S=2048, 50% masks, INT8 gate|up/down, packed KV per layer "
                     "(replace), reuse on every other layer",
            **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in step.items()}}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
