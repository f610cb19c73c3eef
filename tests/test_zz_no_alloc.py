"""The allocation-free csr_add (nacho_gpu_csr_add_f32_noalloc) through the C ABI.

The GPU test compares it with nacho_gpu_csr_add_f32 (bit-exact pos, crd and values) on two
calls in a row, the second on a smaller input, so that state the first call leaves in the
shared static scratch cannot leak into the second; and it checks both against the oracle.
The CPU tests cover the argument checks that run before any device work: the caller's
result capacity and the static scratch's size limit.
"""

import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import assert_csr_equal

NOALLOC_MAX_ITEMS = 250_000_000  # NACHO_NOALLOC_MAX_ITEMS in include/nacho_hip.h


def _desc(lib_mod, rows, cols, pos, crd, val):
    n = crd.numel()
    return lib_mod.CsrDesc(rows, cols, ctypes.c_void_p(pos.data_ptr()), n,
                           ctypes.c_void_p(crd.data_ptr() if n else None),
                           ctypes.c_void_p(val.data_ptr() if n else None), n)


def _noalloc(lib, lib_mod, da, db, rows, cols, cap, device, stream):
    """Run the no-alloc entry point into torch-allocated result buffers of `cap` entries."""
    pos = torch.full((rows + 1,), -7, dtype=torch.int32, device=device)
    crd = torch.full((max(cap, 1),), -7, dtype=torch.int32, device=device)
    val = torch.full((max(cap, 1),), float("nan"), dtype=torch.float32, device=device)
    z = lib_mod.CsrDesc(rows, cols, ctypes.c_void_p(pos.data_ptr()), cap,
                        ctypes.c_void_p(crd.data_ptr()), ctypes.c_void_p(val.data_ptr()), cap)
    rc = lib.nacho_gpu_csr_add_f32_noalloc(ctypes.byref(da), ctypes.byref(db), ctypes.byref(z),
                                           256, 256, ctypes.c_void_p(stream))
    assert rc == 0, lib_mod.error_string(rc)
    assert z.dim_j_offsets == pos.data_ptr() and z.values == val.data_ptr()
    torch.cuda.synchronize()
    n = z.dim_j_length
    assert z.nnz == n
    return pos.cpu().numpy(), crd[:n].cpu().numpy(), val[:n].cpu().numpy()


def _with_alloc(lib, lib_mod, da, db, rows, device, stream):
    """The existing entry point (default allocator); copies the result out and frees it."""
    from nacho_amd import _device

    z = lib_mod.CsrDesc()
    rc = lib.nacho_gpu_csr_add_f32(ctypes.byref(da), ctypes.byref(db), ctypes.byref(z), 256, 256,
                                   ctypes.c_void_p(stream), None)
    assert rc == 0, lib_mod.error_string(rc)
    n = z.dim_j_length
    out = []
    for ptr, count, dtype in ((z.dim_j_offsets, rows + 1, torch.int32),
                              (z.dim_j_indices, n, torch.int32), (z.values, n, torch.float32)):
        t = _device.adopt(ptr, count, dtype, device, stream)  # owns the buffer from here
        torch.cuda.synchronize()
        out.append(t.cpu().numpy())
        del t  # releases it
    return tuple(out)


@pytest.mark.gpu
def test_noalloc_matches_csr_add_twice_second_smaller(gpu):
    from nacho_amd import _device, _lib
    from oracle import oracle

    lib = _lib.load()
    stream = _device.current_stream(gpu)
    from nacho_amd import synth

    # Zipf rows (C2's generator at 2^17 rows), then C1's 4096 x 4096 operands: smaller
    cases = [((1 << 17), (1 << 17), synth.zipf_csr(1 << 17, 21), synth.zipf_csr(1 << 17, 22)),
             (4096, 4096) + synth.c1_operands()]
    for rows, cols, a, b in cases:
        ga = [torch.from_numpy(x).to(gpu) for x in a]
        gb = [torch.from_numpy(x).to(gpu) for x in b]
        da, db = _desc(_lib, rows, cols, *ga), _desc(_lib, rows, cols, *gb)
        cap = len(a[1]) + len(b[1])
        print(f"[gpu] noalloc csr_add rows={rows} nnz=({len(a[1])},{len(b[1])})", flush=True)
        got = _noalloc(lib, _lib, da, db, rows, cols, cap, gpu, stream)
        want = _with_alloc(lib, _lib, da, db, rows, gpu, stream)
        assert_csr_equal(got, want, f"noalloc vs csr_add rows={rows}")
        assert_csr_equal(got, oracle.port_csr_binary("add", rows, *a, *b),
                         f"noalloc vs oracle rows={rows}")


@pytest.mark.gpu
def test_noalloc_calls_from_two_threads_on_two_streams_take_turns(gpu):
    """Two host threads, each on its own stream, call the entry point at the same time
    (ctypes releases the GIL during the call).  Both share the GPU's scratch; the per-GPU
    lock and the drain before return keep every result equal to the allocating entry
    point's."""
    import threading

    from nacho_amd import _device, _lib, synth

    lib = _lib.load()
    rows = cols = 1 << 16
    ops = [(synth.zipf_csr(rows, 31), synth.zipf_csr(rows, 32)),
           (synth.zipf_csr(rows, 33), synth.zipf_csr(rows, 34))]
    descs, wants = [], []
    main = _device.current_stream(gpu)
    for a, b in ops:
        ga = [torch.from_numpy(x).to(gpu) for x in a]
        gb = [torch.from_numpy(x).to(gpu) for x in b]
        da, db = _desc(_lib, rows, cols, *ga), _desc(_lib, rows, cols, *gb)
        descs.append((da, db, ga, gb, len(a[1]) + len(b[1])))
        wants.append(_with_alloc(lib, _lib, da, db, rows, gpu, main))
    streams = [torch.cuda.Stream(gpu) for _ in ops]
    torch.cuda.synchronize()
    results, errors = [[] for _ in ops], []

    def worker(t):
        try:
            da, db, _, _, cap = descs[t]
            # the result buffers are filled on the same stream the call runs on
            with torch.cuda.device(gpu), torch.cuda.stream(streams[t]):
                for _ in range(4):
                    results[t].append(_noalloc(lib, _lib, da, db, rows, cols, cap, gpu,
                                               streams[t].cuda_stream))
        except Exception as e:  # noqa: BLE001 - reported by the main thread
            errors.append(e)

    print(f"[gpu] noalloc two threads rows={rows}", flush=True)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(len(ops))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for t, want in enumerate(wants):
        assert len(results[t]) == 4
        for i, got in enumerate(results[t]):
            assert_csr_equal(got, want, f"thread {t} call {i}")


def test_noalloc_refuses_short_capacity_and_oversized_inputs():
    """Checks that run before any device work (fake device addresses, nothing launched)."""
    from nacho_amd import _lib

    lib = _lib.load()
    fn = lib.nacho_gpu_csr_add_f32_noalloc
    r = ctypes.byref
    a = _lib.CsrDesc(8, 8, ctypes.c_void_p(0x1000), 5, ctypes.c_void_p(0x2000),
                     ctypes.c_void_p(0x3000), 5)
    z = _lib.CsrDesc(8, 8, ctypes.c_void_p(0x4000), 9, ctypes.c_void_p(0x5000),
                     ctypes.c_void_p(0x6000), 9)
    assert fn(r(a), r(a), r(z), 256, 256, None) == -1  # capacity 9 < 5 + 5
    assert z.dim_j_length == 0 and z.nnz == 0 and z.dim_j_offsets == 0x4000
    z = _lib.CsrDesc(8, 8, None, 10, ctypes.c_void_p(0x5000), ctypes.c_void_p(0x6000), 10)
    assert fn(r(a), r(a), r(z), 256, 256, None) == -1  # no offsets buffer
    assert fn(r(a), r(a), None, 256, 256, None) == -1
    half = NOALLOC_MAX_ITEMS // 2 + 1  # two operands just past the limit
    big = _lib.CsrDesc(8, 8, ctypes.c_void_p(0x1000), half, ctypes.c_void_p(0x2000),
                       ctypes.c_void_p(0x3000), half)
    z = _lib.CsrDesc(8, 8, ctypes.c_void_p(0x4000), 2 * half, ctypes.c_void_p(0x5000),
                     ctypes.c_void_p(0x6000), 2 * half)
    rc = fn(r(big), r(big), r(z), 256, 256, None)
    assert rc == -9, _lib.error_string(rc)
    assert "static scratch" in _lib.error_string(-9)
