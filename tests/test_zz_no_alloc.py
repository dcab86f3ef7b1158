"""sdq_quantized_matmul_noalloc against sdq_quantized_matmul_epilogue_raw.

Two calls in a row through the C ABI (the second on a smaller input) plus
two small-M calls (one whose K ranges use the scratch): each output agrees with the allocating entry point's to the
north star's bar (max |d| / max |ref| <= 2e-2, cosine >= 0.9999) and with the
oracle's f64 product on sampled rows, and the library's allocator does not
move during the calls."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import cosine, max_rel_err

pytestmark = pytest.mark.gpu

MAX_REL = 2e-2
MIN_COS = 0.9999


def _gelu64(v):
    c = np.float64(np.float32(0.7978845238685608))
    return 0.5 * v * (1.0 + np.tanh((v + 0.044715 * v ** 3) * c))


def _case(oracle, sdq, stream, M, N, K, bits, seed):
    w = oracle.normals(seed, N * K, 0.02).reshape(N, K)
    q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, bits, stream)
    wq, s, b = oracle.quantize(w, 64, bits)
    deq = oracle.dequantize(wq, s, b, 64, bits)
    xb = sdq.f32_to_bf16_bits(oracle.normals(seed + 1, M * K).reshape(M, K))
    x = sdq.Array.from_numpy(xb, sdq.BFLOAT16)
    bias = oracle.normals(seed + 2, N)
    bias_dev = sdq.Array.from_numpy(bias)
    outs = [sdq.Array.from_numpy(np.zeros((M, N), np.float32)) for _ in range(2)]
    stream.synchronize()
    return dict(M=M, N=N, K=K, bits=bits, q=q, deq=deq, x=x, xv=sdq.bf16_bits_to_f32(xb).reshape(M, K),
                bias=bias, bias_dev=bias_dev, outs=outs)


def _call(sdq, stream, c, fn, out):
    rc = fn(out.device_ptr, sdq.FLOAT32, c["x"].device_ptr, sdq.BFLOAT16, c["K"], c["q"].weight.device_ptr,
            c["q"].scales.device_ptr, c["q"].biases.device_ptr, sdq.FLOAT32, c["M"], c["N"], c["K"], 64,
            c["bits"], c["bias_dev"].device_ptr, sdq.FLOAT32, sdq.ACT_GELU_APPROX, stream.native)
    if rc:
        sdq._check(rc, fn.__name__)


def test_no_alloc_entry_point_matches_the_allocating_one(oracle, sdq, stream):
    L = sdq.lib()
    cases = [
        (1536, 12288, 3072, 4, 4000),  # config-2 fc1: split K through the fixed scratch
        (300, 2048, 4096, 8, 4010),    # smaller: split K again, fewer partial tiles
        (8, 4096, 3072, 4, 4020),      # small M: no scratch at all
        (24, 2048, 8192, 8, 4030),     # small M, x too large for one block: K ranges through the scratch
        (48, 6144, 4096, 4, 4040),     # 64-row tiles: split K through the scratch
    ]
    built = [_case(oracle, sdq, stream, *c) for c in cases]
    active0, cache0 = sdq.active_memory(), sdq.cache_memory()
    for c in built:
        print(f"noalloc M={c['M']} N={c['N']} K={c['K']} bits={c['bits']}", flush=True)
        _call(sdq, stream, c, L.sdq_quantized_matmul_noalloc, c["outs"][0])
    stream.synchronize()
    assert sdq.active_memory() == active0 and sdq.cache_memory() == cache0
    for c in built:
        _call(sdq, stream, c, L.sdq_quantized_matmul_epilogue_raw, c["outs"][1])
    stream.synchronize()
    for c in built:
        got, ref = c["outs"][0].to_numpy(), c["outs"][1].to_numpy()
        err, cos = max_rel_err(got, ref), cosine(got, ref)
        assert err <= MAX_REL and cos >= MIN_COS, (c["M"], err, cos)
        pick = np.unique(np.linspace(0, c["M"] - 1, min(32, c["M"])).astype(int))
        want = _gelu64(c["xv"][pick].astype(np.float64) @ c["deq"].astype(np.float64).T + c["bias"])
        err, cos = max_rel_err(got[pick], want), cosine(got[pick], want)
        assert err <= MAX_REL and cos >= MIN_COS, (c["M"], err, cos)
    # The scratch keeps the last call's contents; a repeat gives the same bits.
    _call(sdq, stream, built[1], L.sdq_quantized_matmul_noalloc, built[1]["outs"][1])
    stream.synchronize()
    assert np.array_equal(built[1]["outs"][1].to_numpy(), built[1]["outs"][0].to_numpy())


def test_no_alloc_entry_point_validates(sdq):
    L = sdq.lib()
    rc = L.sdq_quantized_matmul_noalloc(None, sdq.FLOAT32, None, sdq.BFLOAT16, 64, None, None, None,
                                        sdq.FLOAT32, 4, 64, 64, 48, 4, None, 0, 0, None)
    assert rc != 0
    with pytest.raises(sdq.Error, match="group size 64 or 128, got 48"):
        sdq._check(rc, "noalloc")
