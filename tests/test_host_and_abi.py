"""CPU tests: the C-ABI library loads and exports every entry point of
include/shadowinfer_hip.h, argument validation fails cleanly without a GPU,
and the host-side logic of the Python mirror (codes <-> map, CPU plans,
grouping rules, validation and error behaviour) matches the reference."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import oracle as O
from shadowinfer_amd import _native, get_kernel_status
from shadowinfer_amd.ffn_optimizer import INT8Linear, quantize_ffn_modules
from shadowinfer_amd.shadowkv import (PRECISION_CODES, PackedKVCache, PrecisionPlan, codes_to_map,
                                      map_to_codes, packed_attention)
from shadowinfer_amd.shadowkv.packed_kv_cache import _pack_codes_from_map
from shadowinfer_amd.utils import Quantizer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "shadowinfer_hip.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(si_[a-z0-9_]+)\s*\(", text)))


# ------------------------------------------------------------------- ABI
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_native.LIB_PATH)
    declared = _header_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(_native.EXPORTED_SYMBOLS) == declared
    # every extern "C" entry point defined in the sources is declared (and bound)
    csrc = os.path.join(ROOT, "shadow-infer_amd", "csrc")
    defined = set()
    for f in os.listdir(csrc):
        if f.endswith(".hip"):
            defined |= set(re.findall(r'extern "C"[^(]*?\b(si_[a-z0-9_]+)\s*\(',
                                      open(os.path.join(csrc, f)).read()))
    assert defined == set(declared), sorted(defined ^ set(declared))


def test_abi_version_and_status():
    version = int(re.search(r"#define SI_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert _native.load().si_abi_version() == version
    st = get_kernel_status()
    assert st["hip_extensions_loaded"] and st["abi_version"] == version
    assert st["cpu_fallback"] is False and st["kv_pack_kernel"] == "hip"


def test_status_carries_the_reference_registry_keys(monkeypatch):
    """Every key of the reference's get_kernel_status (kernels/__init__.py:63-70,
    78-87) with its type; the reference's caller reads
    ['sparse_gemm_kernel'] (ffn_optimizer_agent.py:1170), which this library
    does not provide, so it must not read "cuda" there; the
    SHADOWINFER_FORCE_CPU_KERNELS switch (dispatcher.py:46-49) is reported and
    refused with a clear error, since there is no CPU path."""
    monkeypatch.delenv("SHADOWINFER_FORCE_CPU_KERNELS", raising=False)
    st = get_kernel_status()
    ref_keys = {"cuda_available", "cuda_extensions_loaded", "int8_kernel", "int4_kernel",
                "sparse_gemm_kernel", "fused_attention_kernel", "autotune_cache_entries",
                "force_cpu"}
    assert ref_keys <= set(st)
    assert isinstance(st["cuda_available"], bool) and isinstance(st["cuda_extensions_loaded"], bool)
    assert st["cuda_available"] == torch.cuda.is_available()
    assert st["cuda_extensions_loaded"] is True
    assert st["int8_kernel"] == st["int4_kernel"] == st["fused_attention_kernel"] == "hip"
    assert st["sparse_gemm_kernel"] == "unavailable"
    assert st["autotune_cache_entries"] == 0 and st["force_cpu"] is False
    monkeypatch.setenv("SHADOWINFER_FORCE_CPU_KERNELS", "1")
    assert get_kernel_status()["force_cpu"] is True
    with pytest.raises(RuntimeError, match="SHADOWINFER_FORCE_CPU_KERNELS"):
        Quantizer.quantize_int8(torch.ones(2, 4))
    with pytest.raises(RuntimeError, match="SHADOWINFER_FORCE_CPU_KERNELS"):
        _native.call("si_act_quant_i8", 1, 9, 4, 4, 1, 1, None)
    monkeypatch.setenv("SHADOWINFER_FORCE_CPU_KERNELS", "0")
    assert get_kernel_status()["force_cpu"] is False


def test_argument_validation_needs_no_device():
    """Invalid arguments are rejected before any HIP call, with a message."""
    lib = _native.load()
    null = None
    table = _native.table16([None] * 16)
    rc = lib.si_kv_pack(1, 1, 2, 1, 2, 8, 64, 24, 1, 1, table, null)  # 24 does not divide 64
    assert rc == 1 and b"group" in lib.si_last_error()
    assert lib.si_kv_pack(1, 1, 7, 1, 2, 8, 64, 16, 1, 1, table, null) == 1  # bad dtype
    assert lib.si_act_quant_i8(1, 9, 4, 4, 1, 1, null) == 1
    ws = _native.size_query("si_plan_workspace_bytes", 100)
    assert lib.si_plan_scan(1, null, 100, 1, 1, 1, 1, ws - 1, null) == 1
    assert b"workspace" in lib.si_last_error()
    rc = lib.si_attn_packed_fwd(1, 2, 1, 1, 8, 96, 1, 1, table, 2, 8, 16, ctypes.c_float(0.1), 1, 0,
                                1, 1 << 20, null)
    assert rc == 1 and b"head_dim" in lib.si_last_error()
    ws = _native.size_query("si_attn_workspace_bytes", 2, 64)
    rc = lib.si_attn_packed_fwd(16, 2, 1, 2, 8, 64, 1, 1, table, 2, 64, 16, ctypes.c_float(0.1), 16, 0,
                                16, ws - 1, null)
    assert rc == 1 and b"workspace" in lib.si_last_error()
    rc = lib.si_attn_packed_fwd(16, 2, 1, 2, 8, 64, 1, 1, table, 2, 64, 16, ctypes.c_float(0.1), 24, 0,
                                16, ws, null)  # out 8-byte aligned: the staged rows store 16 bytes
    assert rc == 1 and b"16-byte aligned" in lib.si_last_error()
    assert lib.si_int4_unpack_rows(1, 1, 2, 5, 1, null) == 1  # 2 bytes hold at most 4 codes
    with pytest.raises(ValueError, match="si_kv_unpack"):
        _native.call("si_kv_unpack", 1, 1, table, 2, 1, 1, 1, 64, 48, 1, 1, None)


def test_workspace_queries():
    assert _native.size_query("si_attn_workspace_bytes", 32, 8192) >= 32 * 8192 * 4
    # small M streams the weight with K split inside the block: no partials
    assert _native.size_query("si_gemm_workspace_bytes", 16, 11008, 4096) == 0
    assert _native.size_query("si_gemm_workspace_bytes", 2048, 11008, 4096) == 0
    # 64 rows x 11008 columns fill 172 CUs with 64x64 tiles: no K split
    assert _native.size_query("si_gemm_workspace_bytes", 64, 11008, 4096) == 0
    # the 4096-column down projection (K = 11008) has 64 such tiles and splits K
    # in four: int32 partials [4, M, N]
    assert _native.size_query("si_gemm_workspace_bytes", 48, 4096, 11008) == 4 * 48 * 4096 * 4
    n = 8192 * 32
    assert _native.size_query("si_admit_workspace_bytes", n) >= 5 * n
    assert _native.size_query("si_int8_linear_workspace_bytes", 16, 4096, 11008) >= 16 * 4096


# ------------------------------------------------------- codes and plans
def test_map_to_codes_and_back_match_reference_semantics():
    pm = {0: {0: "fp32", 2: "evicted"}, 1: {1: "INT8"}, 2: {0: "int4", 1: "fp16", 2: "fp32"},
          4: {2: "evicted"}}
    codes = map_to_codes(pm, 5, 3)
    assert codes.dtype == torch.int8 and codes.shape == (5, 3)
    np.testing.assert_array_equal(codes.numpy(), O.map_to_codes(pm, 5, 3))
    back = codes_to_map(codes)
    assert back[0] == {0: "fp32", 1: "fp16", 2: "evicted"} and back[3] == {0: "fp16", 1: "fp16", 2: "fp16"}
    with pytest.raises(ValueError):
        map_to_codes({0: {0: "bf16"}}, 1, 1, strict=True)
    assert int(map_to_codes({0: {0: "bf16"}}, 1, 1, strict=False)[0, 0]) == PRECISION_CODES["fp16"]
    with pytest.raises(ValueError):
        codes_to_map(torch.tensor([[7]], dtype=torch.int8))


def test_cpu_plan_matches_oracle():
    rng = np.random.default_rng(3)
    for S, H in ((1, 1), (5, 3), (64, 4), (300, 7)):
        codes = rng.integers(-1, 6, size=(S, H)).astype(np.int8)
        mask = {(int(t), int(h)): bool(rng.random() < 0.4) for t in range(S) for h in range(H)}
        mask[(S + 3, 0)] = True  # out of range -> ignored
        plan = PrecisionPlan.from_codes(torch.from_numpy(codes), reuse_mask=mask)
        ref = O.plan_from_codes(codes, mask)
        assert plan.groups == ref["groups"]
        for p in ("fp32", "fp16", "int8", "int4"):
            np.testing.assert_array_equal(plan.flat_indices[p].numpy(), ref["flat_indices"][p])
        assert plan.evicted_entries == ref["evicted_entries"]
        assert plan.reuse_entries == ref["reuse_entries"]
        assert plan.fingerprint == ref["fingerprint"]
        assert plan.reuse_set() == set(ref["reuse_entries"])


def test_plan_build_equals_from_codes_and_is_immutable():
    names = ("fp32", "fp16", "int8", "int4")
    pm = {t: {h: names[(t + h) % 4] for h in range(3)} for t in range(6)}
    built = PrecisionPlan.build(pm, 6, 3, reuse_mask={(1, 1): True})
    other = PrecisionPlan.from_codes(map_to_codes(pm, 6, 3), reuse_mask={(1, 1): True})
    assert built.groups == other.groups and built.fingerprint == other.fingerprint
    with pytest.raises(AttributeError):
        built.seq_len = 3
    with pytest.raises(ValueError):
        PrecisionPlan.from_codes(torch.zeros(4, dtype=torch.int8))
    with pytest.raises(ValueError):
        PrecisionPlan.from_codes(torch.zeros(0, 3, dtype=torch.int8))
    with pytest.raises(ValueError):
        PrecisionPlan.build({1: {1: "bf16"}}, 2, 2, strict=True)
    with pytest.raises(ValueError):
        built.device_grouping()  # a CPU plan cannot drive a device pack


def test_pack_map_grouping_rules():
    rng = np.random.default_rng(9)
    names = ["fp32", "FP16", "int8", "int4", "evicted", "bf16", "weird"]
    pm = {t: {h: names[rng.integers(0, len(names))] for h in range(4) if rng.random() < 0.8}
          for t in range(20) if rng.random() < 0.9}
    np.testing.assert_array_equal(_pack_codes_from_map(pm, 20, 4).reshape(20, 4),
                                  O.pack_map_to_codes(pm, 20, 4))


# ----------------------------------------------------- error behaviour
def test_cpu_tensors_fail_loudly():
    k = torch.randn(1, 2, 4, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        PackedKVCache.pack(k, k, {})
    with pytest.raises(RuntimeError, match="HIP device"):
        Quantizer.quantize_int8(k)
    layer = INT8Linear(torch.zeros(64, 32, dtype=torch.int8), torch.ones(32))
    with pytest.raises(RuntimeError, match="HIP device"):
        layer(torch.randn(3, 64))
    with pytest.raises(RuntimeError, match="HIP device"):
        INT8Linear.from_linear(nn.Linear(8, 8))


def test_rope_pack_rejects_bad_tables_before_any_launch():
    """pack_projection reads cos/sin [S, D] in qkv's dtype for every token: a
    short table or one of another dtype is a ValueError (a short table would be
    read past its end, an fp32 one as bf16 pairs); well-formed CPU tensors are
    the usual no-CPU-implementation error."""
    B, S, H, D = 1, 6, 2, 64
    plan = PrecisionPlan.from_codes(torch.full((S, H), 2, dtype=torch.int8))
    qkv = torch.zeros(B * S, 3 * H * D, dtype=torch.bfloat16)
    good = torch.zeros(S, D, dtype=torch.bfloat16)
    for cos, sin in ((good[: S - 1], good[: S - 1]), (good.float(), good.float()), (good, good[:, :32])):
        with pytest.raises(ValueError, match="cos/sin"):
            PackedKVCache.pack_projection(qkv, cos, sin, B, S, H, D, 16, plan)
    with pytest.raises(ValueError, match="qkv must be"):
        PackedKVCache.pack_projection(qkv[:, : 2 * H * D], good, good, B, S, H, D, 16, plan)
    with pytest.raises(RuntimeError, match="HIP device"):
        PackedKVCache.pack_projection(qkv, good, good, B, S, H, D, 16, plan)


def test_empty_cache_is_safe_without_device():
    """reference tests/test_kv_store.py:528-552 (UT-12.10)."""
    packed = PackedKVCache(1, 2, 8, 64)
    k, v = packed.unpack()
    assert k.shape == (1, 2, 8, 64) and torch.count_nonzero(k) == 0 and torch.count_nonzero(v) == 0
    assert packed.evict({(0, 0)}) == 0
    assert packed.memory_bytes() == 0 and packed.resident_bytes() == 0
    assert packed.packed_data == {}
    assert packed.apply_reuse_mask(PackedKVCache(1, 2, 8, 64), {(0, 0): True}, return_stats=True) == \
        {"applied": 0, "skipped_precision": 0}
    with pytest.raises(ValueError):
        packed.apply_reuse_mask(PackedKVCache(1, 2, 8, 32), {(0, 0): True})
    assert "PackedKVCache(batch=1" in repr(packed)


def test_int8_linear_validation_and_accounting():
    """reference tests/test_int8_ffn.py:114-152."""
    layer = INT8Linear(torch.zeros(128, 96, dtype=torch.int8), torch.ones(96), bias=torch.zeros(96))
    assert layer(torch.empty(0, 128)).shape == (0, 96)
    with pytest.raises(ValueError):
        layer(torch.randn(4, 127))
    with pytest.raises(ValueError):
        INT8Linear(torch.zeros(128, dtype=torch.int8), torch.ones(96))
    with pytest.raises(ValueError):
        INT8Linear(torch.zeros(128, 96, dtype=torch.int8), torch.ones(95))
    with pytest.raises(ValueError):
        INT8Linear(torch.zeros(128, 96, dtype=torch.int8), torch.ones(96), bias=torch.zeros(95))
    with pytest.raises(ValueError):
        INT8Linear(torch.zeros(128, 96, dtype=torch.int16), torch.ones(96))
    assert layer.memory_bytes() == 128 * 96 + 4 * 96 + 4 * 96
    assert layer.dense_equivalent_bytes() == 4 * 128 * 96 + 4 * 96
    nobias = INT8Linear(torch.zeros(128, 96, dtype=torch.int8), torch.ones(96))
    assert nobias.dense_equivalent_bytes() / nobias.memory_bytes() >= 3.8
    assert layer.qweight.dtype == torch.int8 and layer.weight_scale.dtype == torch.float32
    assert set(layer.state_dict()) == {"qweight", "weight_scale", "bias"}
    with pytest.raises(TypeError):
        INT8Linear.from_linear(nn.Conv1d(2, 2, 1))
    assert quantize_ffn_modules(nn.Sequential(nn.Linear(4, 4))) == {"supported": False}


def test_quantizer_host_rules():
    with pytest.raises(ValueError):
        Quantizer.quantize_tensor(torch.randn(10), "int2")
    with pytest.raises(ValueError):
        Quantizer.dequantize_tensor(torch.zeros(10, dtype=torch.int8), None, "int8")
    with pytest.raises(ValueError):
        Quantizer.dequantize_tensor(torch.zeros(10, 2, dtype=torch.int8), None, "int4")
    x = torch.randn(10, 20)
    q, s = Quantizer.quantize_tensor(x, "fp32")
    assert q is x and s is None
    q, s = Quantizer.quantize_tensor(x, "fp16")
    assert q.dtype == torch.float16 and s is None
    q, s = Quantizer.quantize_int8(torch.empty(0))
    assert q.numel() == 0 and float(s) == 1.0
    # the empty round trip: a 0-d scale broadcasts against the empty codes
    d = Quantizer.dequantize_int8(q, s)
    assert d.shape == (0,) and d.dtype == torch.float32
    q4, s4 = Quantizer.quantize_int4(torch.empty(3, 0, 16))
    assert Quantizer.dequantize_int4(q4, s4).shape == (3, 0)
    with pytest.raises(TypeError):
        Quantizer.dequantize_int8(q, torch.tensor(1.0, dtype=torch.float64))
    assert Quantizer.pack_int4(torch.empty(0, dtype=torch.int8)).numel() == 0
    assert Quantizer.unpack_int4(torch.empty(0, dtype=torch.uint8), (2, 3)).shape == (2, 3)


def test_packed_attention_validation():
    cache = PackedKVCache(1, 2, 16, 64)
    with pytest.raises(ValueError):
        packed_attention(torch.randn(1, 3, 8, 64, dtype=torch.bfloat16), cache)
    with pytest.raises(ValueError):
        packed_attention(torch.randn(8, 64, dtype=torch.bfloat16), cache)
    with pytest.raises(TypeError):
        packed_attention(torch.randn(1, 2, 8, 64), cache)


def test_step_and_copy_entry_points_reject_bad_arguments():
    """The denoising-step row kernels, the bucket-order copies, the page-run
    writer and the prebuilt-list attention reject invalid arguments before any
    HIP call (status 1 and a message; no device needed)."""
    lib = _native.load()
    null = None
    t4 = _native.table4([None] * 4)
    t16 = _native.table16([None] * 16)
    c5 = (ctypes.c_int64 * 5)(0, 1, 0, 0, 0)
    c4 = (ctypes.c_int64 * 4)(0, 1, 3, 0)
    big = (ctypes.c_int64 * 4)(0, 9, 9, 0)   # 18 listed entries in an 8 x 2 matrix
    grow = (ctypes.c_int64 * 4)(0, 2, 3, 0)  # more rows than the old bucket
    l4 = _native.table4([None, 16, 16, None])
    k_only = _native.table16([None] * 8 + [16, 16, None, None] + [None] * 4)  # int8 without scales
    f = ctypes.c_float
    rows = 64 * lib.si_kv_evict_chunk_words()
    assert rows in (128, 256)
    assert lib.si_kv_evict_chunks(c4) == 2 and lib.si_kv_evict_chunks(null) == -1
    assert lib.si_kv_evict_chunks((ctypes.c_int64 * 4)(0, -1, 0, 0)) == -1
    assert lib.si_kv_evict_chunks((ctypes.c_int64 * 4)(rows, rows + 1, 0, 1)) == 4
    checks = [
        # K not a multiple of 8 / above the register budget / q without scale
        (lambda: lib.si_rmsnorm_rows(16, 2, 4, 12, 16, f(1e-5), 16, null, null, null), b"multiple of 8"),
        (lambda: lib.si_rmsnorm_rows(16, 2, 4, 32768, 16, f(1e-5), 16, null, null, null), b"multiple of 8"),
        (lambda: lib.si_rmsnorm_rows(16, 2, 4, 64, 16, f(1e-5), null, 16, null, null), b"together"),
        (lambda: lib.si_rmsnorm_rows(16, 9, 4, 64, 16, f(1e-5), 16, null, null, null), b"dtype"),
        (lambda: lib.si_rmsnorm_rows(8, 2, 4, 64, 16, f(1e-5), 16, null, null, null), b"aligned"),
        (lambda: lib.si_rope_split(16, 2, 1, 8, 4, 96, 16, 16, 16, 16, 16, null), b"head_dim"),
        (lambda: lib.si_rope_split(16, 2, 1, 8, 4, 64, 16, 16, null, 16, 16, null), b"NULL"),
        (lambda: lib.si_swiglu_quant(16, 2, 4, 12, null, 16, 16, null), b"multiple of 8"),
        (lambda: lib.si_swiglu_quant(16, 2, 4, 64, null, null, 16, null), b"NULL"),
        (lambda: lib.si_row_argmax_conf(16, 2, 4, 0, 16, 16, null), b"shape"),
        (lambda: lib.si_row_argmax_conf(16, 7, 4, 8, 16, 16, null), b"dtype"),
        (lambda: lib.si_kv_reuse_flat(t4, c5, t16, 8, 1, 1, t16, 8, 1, 2, 1, 64, 48, 2, null, null), b"group"),
        (lambda: lib.si_kv_reuse_flat(t4, c5, t16, 8, 1, 1, t16, 8, null, 2, 1, 64, 16, 2, null, null), b"NULL"),
        (lambda: lib.si_kv_compact_flat(1, t16, t4, c5, t16, 8, 2, 1, 64, 16, 9, null), b"scale dtype"),
        # evict passes: missing arguments, inconsistent sizes, absent scale tensors
        (lambda: lib.si_kv_evict_count(16, t4, c4, null, 8, 2, 16, 16, 16, 16, null), b"NULL"),
        (lambda: lib.si_kv_evict_count(16, t4, c4, 16, 8, 2, 16, 16, 16, 16, null), b"NULL list"),
        (lambda: lib.si_kv_evict_count(16, l4, big, 16, 8, 2, 16, 16, 16, 16, null), b"lists hold"),
        (lambda: lib.si_kv_evict_count(16, l4, c4, 16, 8, 2, 16, 16, 16, null, null), b"bits"),
        (lambda: lib.si_kv_evict_flat(l4, c4, 16, 16, 8, 2, t16, t4, grow, t16, 16, 1, 64, 16, 2, null),
         b"new bucket 1"),
        (lambda: lib.si_kv_evict_flat(l4, c4, 16, 16, 8, 2, t16, t4, c4, k_only, 16, 1, 64, 16, 2, null),
         b"NULL bucket tensor"),
        (lambda: lib.si_kv_evict_flat(l4, c4, 16, 16, 8, 2, t16, t4, c4, t16, 16, 1, 64, 48, 2, null),
         b"group"),
        (lambda: lib.si_page_write_pages(16, 16, 2, 1, 2, 8, 64, 0, 2, 2, 16, t4, 8, null), b"outside"),
        (lambda: lib.si_page_write_pages(16, 16, 2, 1, 2, 64, 64, 0, 2, 5, 16, t4, 8, null), b"precision"),
        (lambda: lib.si_attn_build_lists(1, 1, 2, 64, 16, 7, null), b"workspace"),
        (lambda: lib.si_attn_packed_fwd_built(16, 2, 1, 2, 8, 96, 16, 1 << 20, t16, 2, 64, 16, f(0.1), 16, 0,
                                      0, null), b"head_dim"),
    ]
    for call, word in checks:
        rc = call()
        msg = lib.si_last_error()
        assert rc == 1 and word in msg, (rc, msg, word)
    # zero-sized work is a no-op that succeeds
    assert lib.si_rmsnorm_rows(null, 2, 0, 64, null, f(1e-5), null, null, null, null) == 0
    assert lib.si_swiglu_quant(null, 2, 0, 64, null, null, null, null) == 0
    assert lib.si_rope_split(null, 2, 0, 8, 4, 64, null, null, null, null, null, null) == 0
    assert lib.si_kv_compact_flat(1, t16, t4, c5, t16, 0, 2, 1, 64, 16, 2, null) == 0
    assert lib.si_kv_evict_count(null, null, null, null, 0, 2, null, null, null, null, null) == 0
    assert lib.si_kv_evict_flat(null, null, null, null, 8, 0, null, null, null, null, null, 1, 64, 16,
                                2, null) == 0


def test_token_head_masks_follow_python_membership():
    """The set / dict arguments of evict / apply_reuse_mask become a dense mask
    by the reference's own rule: entry (t, h) is marked when ``(t, h) in items``
    (a set) or ``items.get((t, h))`` is truthy (a dict), whatever the element
    types (packed_kv_cache.py:679-687, 798-814). Both the host extension and the
    item-by-item fallback are checked against that brute-force rule."""
    import numpy as np
    from shadowinfer_amd.shadowkv import _masks

    S, H = 7, 3
    items = {(0, 0), (1, 2), (True, False), (2.0, 1), (3.5, 1), (np.int64(4), np.int32(2)),
             (6, 3), (-1, 0), (7, 0), (10 ** 30, 1), ("a", 1), (5,), (5, 1, 0), "x",
             (float("nan"), 0), (np.float32(6.0), 0)}
    as_dict = {k: (i % 3 != 0) for i, k in enumerate(sorted(items, key=repr))}
    as_dict[(3, 0)] = 0
    as_dict[(3, 1)] = "yes"
    for container, is_dict in ((items, False), (frozenset(items), False), (as_dict, True)):
        want = np.array([bool(container.get((t, h), False)) if is_dict else ((t, h) in container)
                         for t in range(S) for h in range(H)], dtype=np.uint8)
        got = _masks.token_head_mask(container, S, H, is_dict=is_dict)
        got = np.zeros(S * H, np.uint8) if got is None else got
        np.testing.assert_array_equal(got, want)
        slow = np.zeros(S * H, np.uint8)
        _masks._mark_python(container, S, H, slow, is_dict)
        np.testing.assert_array_equal(slow, want)
    assert _masks.token_head_mask(set(), S, H) is None


def test_token_head_masks_evaluate_values_only_for_pairs(recwarn):
    """A dict value's truthiness is evaluated only for keys that are in-range
    (t, h) pairs: a value whose __bool__ raises under an irrelevant key is never
    touched (the reference looks values up only for entries of the cache). Under
    a relevant key it raises, as ``if reuse_mask.get(entry)`` would. numpy bool
    elements equal 0 / 1, as in Python, and raise no DeprecationWarning."""
    import warnings

    import numpy as np
    from shadowinfer_amd.shadowkv import _masks

    class Boom:
        def __bool__(self):
            raise RuntimeError("truthiness evaluated")

    S, H = 4, 2
    d = {(1, 1): True, (9, 0): Boom(), ("x", 0): Boom(), (0, 5): Boom(), (2,): Boom(),
         (np.True_, np.False_): 1, (np.int64(3), np.bool_(True)): np.True_}
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        got = _masks.token_head_mask(d, S, H, is_dict=True)
        slow = np.zeros(S * H, np.uint8)
        _masks._mark_python(d, S, H, slow, True)
        s = _masks.token_head_mask({(np.True_, np.True_), (np.bool_(False), 1)}, S, H)
    want = np.zeros(S * H, np.uint8)
    want[[1 * H + 1, 1 * H + 0, 3 * H + 1]] = 1
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(slow, want)
    np.testing.assert_array_equal(np.nonzero(s)[0], [0 * H + 1, 1 * H + 1])
    with pytest.raises(RuntimeError, match="truthiness"):
        _masks.token_head_mask({(0, 0): Boom()}, S, H, is_dict=True)


def test_map_to_codes_random_maps_match_the_dense_rule():
    """The sparse host walk of map_to_codes against the oracle's dense grid
    walk (precision_plan.py:30-55) on random maps whose keys are ints, floats,
    bools, numpy integers and out-of-grid values, with mixed-case and unknown
    names; the first unknown name in (token, head) order is the one reported.
    codes_to_map inverts it exactly on random code matrices."""
    import numpy as np
    from shadowinfer_amd.shadowkv.precision_plan import codes_to_map, map_to_codes

    rng = np.random.default_rng(11)
    names = ["fp32", "FP16", "Int8", "int4", "evicted", "bf16", "fp8", 3, None]
    for trial in range(40):
        S, H = int(rng.integers(1, 12)), int(rng.integers(1, 6))
        pm = {}
        for _ in range(int(rng.integers(0, 2 * S))):
            t = int(rng.integers(-2, S + 2))
            tk = [t, float(t), np.int64(t)][int(rng.integers(0, 3))] if t != 1 else [1, True][int(rng.integers(0, 2))]
            row = pm.setdefault(tk, {})
            for _ in range(int(rng.integers(0, H + 2))):
                h = int(rng.integers(-1, H + 1))
                hk = [h, float(h) + [0.0, 0.5][int(rng.integers(0, 2))], np.int32(h)][int(rng.integers(0, 3))]
                row[hk] = names[int(rng.integers(0, 5 if trial % 2 else len(names)))]
        for strict in (True, False):
            try:
                want = O.map_to_codes(pm, S, H, strict=strict)
            except ValueError as e:
                with pytest.raises(ValueError) as got:
                    map_to_codes(pm, S, H, strict=strict)
                assert str(got.value) == str(e)
                continue
            np.testing.assert_array_equal(map_to_codes(pm, S, H, strict=strict).numpy(), want)
        codes = rng.integers(0, 5, size=(S, H)).astype(np.int8)
        back = codes_to_map(torch.from_numpy(codes))
        assert list(back) == list(range(S)) and all(list(r) == list(range(H)) for r in back.values())
        np.testing.assert_array_equal(map_to_codes(back, S, H).numpy(), codes)
