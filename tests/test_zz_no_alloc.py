"""si_int8_linear_forward_noalloc: the INT8Linear forward with its workspace in
the library's per-device scratch array, called through the C ABI and compared
with si_int8_linear_forward (caller workspace) on the same inputs: bit-exact
outputs on consecutive calls (the second with a smaller input, then a shape
whose GEMM splits K through int32 partials), and a clear rejection of a shape
whose workspace exceeds the scratch."""

import pytest
import torch

from shadowinfer_amd import _native


def _layer(dev, N, K, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn(N, K, generator=g, device=dev) * 0.02
    q = torch.empty(N, K, dtype=torch.int8, device=dev)
    s = torch.empty(N, dtype=torch.float32, device=dev)
    _native.call("si_weight_quant_i8", w.data_ptr(), N, K, q.data_ptr(), s.data_ptr(),
                 _native.stream(dev))
    return q, s


def _forward(x, q, s, bias, noalloc):
    dev = x.device
    M, K = x.shape
    N = q.shape[0]
    out = torch.full((M, N), float("nan"), dtype=x.dtype, device=dev)
    args = (x.data_ptr(), _native.dtype_code(x.dtype), M, K, N, q.data_ptr(), s.data_ptr(),
            _native.ptr(bias), out.data_ptr())
    if noalloc:
        _native.call("si_int8_linear_forward_noalloc", *args, _native.stream(dev))
    else:
        ws_bytes = _native.size_query("si_int8_linear_workspace_bytes", M, K, N)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        _native.call("si_int8_linear_forward", *args, ws.data_ptr(), ws_bytes,
                     _native.stream(dev))
    return out


@pytest.mark.gpu
def test_noalloc_forward_equals_workspace_forward(dev):
    cases = [(256, 4096, 11008, torch.bfloat16, True),     # 128x128 tiles
             (16, 4096, 11008, torch.bfloat16, False),     # smaller: 64x64 tiles
             (128, 11008, 4096, torch.float16, True)]      # K split in four (int32 partials)
    for i, (M, K, N, dt, with_bias) in enumerate(cases):
        print(f"noalloc case {i}: M={M} K={K} N={N} {dt}", flush=True)
        need = _native.size_query("si_int8_linear_workspace_bytes", M, K, N)
        assert need <= 32 << 20
        q, s = _layer(dev, N, K, seed=i)
        g = torch.Generator(device=dev).manual_seed(100 + i)
        x = torch.randn(M, K, generator=g, device=dev).to(dt)
        bias = torch.randn(N, generator=g, device=dev) if with_bias else None
        want = _forward(x, q, s, bias, noalloc=False)
        got = _forward(x, q, s, bias, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"case {i}"
        assert not torch.isnan(got).any()
    # the last case's workspace holds split-K partials besides the activations
    assert _native.size_query("si_int8_linear_workspace_bytes", 128, 11008, 4096) > \
        128 * 11008 + 128 * 4 + 512


@pytest.mark.gpu
def test_noalloc_rejects_shapes_beyond_the_scratch(dev):
    M, K, N = 8192, 4096, 256                  # quantized activations alone: 32 MiB
    assert _native.size_query("si_int8_linear_workspace_bytes", M, K, N) > 32 << 20
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(N, K, dtype=torch.int8, device=dev)
    s = torch.ones(N, dtype=torch.float32, device=dev)
    out = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="scratch"):
        _native.call("si_int8_linear_forward_noalloc", x.data_ptr(), _native.dtype_code(x.dtype),
                     M, K, N, q.data_ptr(), s.data_ptr(), None, out.data_ptr(),
                     _native.stream(dev))
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())            # nothing was launched
