"""libsdq from several host threads at once.

The reference runs its tests on parallel threads and its error trampoline
relies on the message reaching the thread whose call failed
(crates/sd-tensor/src/mlx.rs:419-470; sd-models/src/mlx/flux.rs:207-224).
The CPU tests here fail calls during argument validation, before any GPU
work, so they run without a GPU; the GPU tests drive streams, arrays, the
allocator and the kernels from several threads, and the allocator's ordering
of a block's reuse after a reader on another stream."""
from __future__ import annotations

import threading

import numpy as np
import pytest

from conftest import cosine, max_rel_err


def _run_threads(n, fn):
    errors = []

    def wrap(i):
        try:
            fn(i)
        except BaseException as e:  # noqa: BLE001 - reported to the main thread
            errors.append((i, e))

    ts = [threading.Thread(target=wrap, args=(i,)) for i in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors


def test_each_thread_receives_its_own_error_message(sdq):
    # A bad group size fails validation with a message naming it; 8 threads
    # with 8 different sizes, 200 calls each, must never see another's text.
    L = sdq.lib()

    def worker(i):
        gs = 1000 + i
        for _ in range(200):
            rc = L.sdq_quantized_matmul_raw(None, sdq.FLOAT32, None, sdq.BFLOAT16, 64, None, None, None,
                                            sdq.FLOAT32, 1, 64, 64, gs, 4, None)
            assert rc != 0
            msg = sdq._take_last_error()
            assert msg is not None and f"group size {gs} " in msg, msg

    _run_threads(8, worker)


def test_a_success_clears_the_stale_message_per_thread(sdq):
    # mlx.rs:459-465: a successful call clears any stale message.
    L = sdq.lib()

    def worker(i):
        for _ in range(100):
            L.sdq_quantized_matmul_raw(None, sdq.FLOAT32, None, sdq.BFLOAT16, 64, None, None, None,
                                       sdq.FLOAT32, 1, 64, 64, 7, 4, None)
            with pytest.raises(sdq.Error):
                sdq._check(1, "x")
            sdq._check(0, "ok")
            assert sdq._take_last_error() is None

    _run_threads(4, worker)


def test_cpu_stream_handles_from_many_threads(sdq):
    # Handles are created and freed concurrently; ops on them fail loudly.
    def worker(i):
        for _ in range(200):
            s = sdq.Stream.cpu()
            with pytest.raises(sdq.Error, match="no CPU backend"):
                s.synchronize()
            del s

    _run_threads(8, worker)


@pytest.mark.gpu
def test_threads_with_their_own_streams(sdq, oracle):
    # Each thread quantizes and multiplies on a stream of its own while the
    # others do the same; every result matches the oracle.
    N, K = 512, 1024

    def worker(i):
        s = sdq.Stream.new()
        w = oracle.normals(3000 + i, N * K, 0.02).reshape(N, K)
        q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, 4 if i % 2 else 8, s)
        wq, sc, b = oracle.quantize(w, 64, q.bits)
        deq = oracle.dequantize(wq, sc, b, 64, q.bits)
        for M in (1, 7, 40, 300):
            x = oracle.normals(3100 + i + M, M * K).reshape(M, K)
            bits = sdq.f32_to_bf16_bits(x)
            y = q.matmul(sdq.Array.from_numpy(bits, sdq.BFLOAT16), s).to_numpy()
            want = sdq.bf16_bits_to_f32(bits).reshape(M, K).astype(np.float64) @ deq.astype(np.float64).T
            assert max_rel_err(y, want) <= 2e-2 and cosine(y, want) >= 0.9999
        s.synchronize()
        del s

    _run_threads(6, worker)


@pytest.mark.gpu
def test_block_reuse_waits_for_a_reader_on_another_stream(sdq, oracle):
    # x is produced on stream A and read by a long matmul on stream B; x is
    # then freed and a block of the same size is at once allocated and
    # overwritten on A.  The allocator must order that reuse after B's read:
    # B's result still matches the original x.
    a, b = sdq.Stream.new(), sdq.Stream.new()
    N, K, M = 8192, 8192, 2048
    w = oracle.normals(3200, N * K, 0.02).reshape(N, K)
    q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, 4, a)
    a.synchronize()
    src = oracle.normals(3201, M * K).reshape(M, K)
    x = sdq.Array.from_numpy(src).astype(sdq.BFLOAT16, a)      # produced on A
    other = sdq.Array.from_numpy(np.full((M, K), 7.0, np.float32))
    wq, sc, bb = oracle.quantize(w, 64, 4)
    deq = oracle.dequantize(wq, sc, bb, 64, 4)
    pick = np.linspace(0, M - 1, 16).astype(int)
    xs = sdq.bf16_bits_to_f32(sdq.f32_to_bf16_bits(src[pick])).reshape(len(pick), K)
    want = xs.astype(np.float64) @ deq.astype(np.float64).T
    for trial in range(3):
        print(f"reuse trial {trial}", flush=True)
        y = q.matmul(x, b)                                      # read on B (long)
        del x
        z = other.astype(sdq.BFLOAT16, a)                       # same size, on A
        assert np.all(sdq.bf16_bits_to_f32(z.to_numpy()) == 7.0)
        got = y.to_numpy()
        assert max_rel_err(got[pick], want) <= 2e-2 and cosine(got[pick], want) >= 0.9999, trial
        del z
        x = sdq.Array.from_numpy(src).astype(sdq.BFLOAT16, a)
    a.synchronize()
    b.synchronize()


@pytest.mark.gpu
def test_freed_stream_leaves_no_dead_handle_behind(sdq, oracle):
    # An array made on a stream that is then freed can still be used and
    # freed; its block is reused on another stream without touching the
    # destroyed stream.
    s = sdq.Stream.new()
    x = sdq.Array.from_numpy(np.ones((256, 256), np.float32)).astype(sdq.BFLOAT16, s)
    s.synchronize()
    del s
    t = sdq.Stream.new()
    y = x.astype(sdq.FLOAT32, t)
    assert np.all(y.to_numpy() == 1.0)
    del x
    z = sdq.Array.from_numpy(np.full((256, 256), 2.0, np.float32)).astype(sdq.BFLOAT16, t)
    assert np.all(sdq.bf16_bits_to_f32(z.to_numpy()) == 2.0)
    t.synchronize()
