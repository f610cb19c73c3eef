"""CPU oracle for the nacho GPU path — TEST INFRASTRUCTURE, never the product.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and
only as the checker.  Two independent kinds of reference live here:

1. `port_*`: ctypes bindings to nacho_oracle.c, the C restatement of the reference's
   generated CPU pipeline (per-thread merge-path partition, count, serial scan, write).
   Each function's file:line anchors are in nacho_oracle.c.
2. `closed_*`: numpy closed forms of the same results, derived from the mathematics only
   (sorted union / intersection of coordinate keys, lexsort + run-length reduce), used to
   pin (1) — a mistake in the partitioning, lattice or scan of (1) fails against (2).

Parity status of each function (how it is pinned) is recorded in the test modules and in
the repository's design notes: csr/coo/coo3/csf union and intersection are pinned by the
closed forms, by scipy, by brute force on tiny inputs and by the reference's own smoke
cases (tests/smoke.py semantics); dcsr union / intersection by the DCSR closed form over the
expanded CSR matrices; csr_add3 by the three-way closed form; spgemm and sssmm are
pinned by float64 scipy products; the csf3 / coo3 inner products by the key-intersection
closed form and by brute force over coordinate dictionaries.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIBRARY = ORACLE_DIR / "liboracle.so"

_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_f32p = ctypes.POINTER(ctypes.c_float)

_lib = None


def build() -> Path:
    """Compile nacho_oracle.c with gcc (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-C", str(ORACLE_DIR), "liboracle.so"], check=True)
    return LIBRARY


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        lib.oracle_free.argtypes = [ctypes.c_void_p]
        lib.oracle_free.restype = None
        lib.oracle_default_threads.restype = ctypes.c_int
        lib.oracle_csr_binary.restype = ctypes.c_int
        lib.oracle_csr_binary.argtypes = [
            ctypes.c_int, ctypes.c_int, _i32p, _i32p, _f32p, ctypes.c_int, _i32p, _i32p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.POINTER(_i32p), ctypes.POINTER(_i32p),
            ctypes.POINTER(_f32p), ctypes.POINTER(ctypes.c_int)]
        lib.oracle_coo_binary.restype = ctypes.c_int
        lib.oracle_coo_binary.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.POINTER(_i32p), _f32p, ctypes.c_int,
            ctypes.POINTER(_i32p), _f32p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_i32p),
            ctypes.POINTER(_f32p), ctypes.POINTER(ctypes.c_int)]
        lib.oracle_csf3_union.restype = ctypes.c_int
        lib.oracle_csf3_union.argtypes = (
            [_i32p, ctypes.c_int, _i32p, _i32p, ctypes.c_int, _i32p, _i32p, _f32p, ctypes.c_int]
            * 2 + [ctypes.POINTER(_i32p)] * 5 + [ctypes.POINTER(_f32p)]
            + [ctypes.POINTER(ctypes.c_int)] * 3)
        lib.oracle_csr_add3.restype = ctypes.c_int
        lib.oracle_csr_add3.argtypes = (
            [ctypes.c_int] + [_i32p, _i32p, _f32p] * 3
            + [ctypes.POINTER(_i32p), ctypes.POINTER(_i32p), ctypes.POINTER(_f32p),
               ctypes.POINTER(ctypes.c_int)])
        lib.oracle_sssmm.restype = ctypes.c_int
        lib.oracle_sssmm.argtypes = (
            [ctypes.c_int, ctypes.c_int] + [_i32p, _i32p, _f32p] * 3
            + [_i32p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_i32p), ctypes.POINTER(_i32p),
               ctypes.POINTER(_f32p), ctypes.POINTER(ctypes.c_int)])
        lib.oracle_dcsr_binary.restype = ctypes.c_int
        lib.oracle_dcsr_binary.argtypes = (
            [ctypes.c_int] + [_i32p, ctypes.c_int, _i32p, _i32p, _f32p] * 2
            + [ctypes.POINTER(_i32p)] * 3 + [ctypes.POINTER(_f32p)]
            + [ctypes.POINTER(ctypes.c_int)] * 2)
        lib.oracle_csf3_union_mt.restype = ctypes.c_int
        lib.oracle_csf3_union_mt.argtypes = (
            [_i32p, ctypes.c_int, _i32p, _i32p, ctypes.c_int, _i32p, _i32p, _f32p, ctypes.c_int]
            * 2 + [ctypes.c_int] + [ctypes.POINTER(_i32p)] * 5 + [ctypes.POINTER(_f32p)]
            + [ctypes.POINTER(ctypes.c_int)] * 3)
        lib.oracle_csr_add3_mt.restype = ctypes.c_int
        lib.oracle_csr_add3_mt.argtypes = (
            [ctypes.c_int] + [_i32p, _i32p, _f32p] * 3 + [ctypes.c_int]
            + [ctypes.POINTER(_i32p), ctypes.POINTER(_i32p), ctypes.POINTER(_f32p),
               ctypes.POINTER(ctypes.c_int)])
        lib.oracle_dcsr_binary_mt.restype = ctypes.c_int
        lib.oracle_dcsr_binary_mt.argtypes = (
            [ctypes.c_int] + [_i32p, ctypes.c_int, _i32p, _i32p, _f32p] * 2 + [ctypes.c_int]
            + [ctypes.POINTER(_i32p)] * 3 + [ctypes.POINTER(_f32p)]
            + [ctypes.POINTER(ctypes.c_int)] * 2)
        lib.oracle_csf3_inner.restype = ctypes.c_int
        lib.oracle_csf3_inner.argtypes = (
            [_i32p, ctypes.c_int, _i32p, _i32p, _i32p, _i32p, _f32p] * 2
            + [ctypes.c_int, ctypes.POINTER(ctypes.c_double)])
        lib.oracle_coo3_inner.restype = ctypes.c_int
        lib.oracle_coo3_inner.argtypes = (
            [_i32p, _i32p, _i32p, _f32p, ctypes.c_int] * 2
            + [ctypes.c_int, ctypes.POINTER(ctypes.c_double)])
        lib.oracle_spgemm.restype = ctypes.c_int
        lib.oracle_spgemm.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p, _i32p, _f32p, _i32p, _i32p, _f32p,
            ctypes.c_int, ctypes.POINTER(_i64p), ctypes.POINTER(_i32p), ctypes.POINTER(_f32p),
            ctypes.POINTER(ctypes.c_int64)]
        _lib = lib
    return _lib


def _as(arr, dtype):
    a = np.ascontiguousarray(arr, dtype=dtype)
    if a.size == 0:  # never hand C a null pointer for an empty array
        a = np.zeros(1, dtype=dtype)
    return a


def _ptr(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _take(ptr, n, dtype):
    """Copy n elements from a malloc'd C array into numpy, then free it."""
    lib = load()
    out = np.ctypeslib.as_array(ptr, shape=(max(n, 1),))[:n].astype(dtype, copy=True)
    lib.oracle_free(ctypes.cast(ptr, ctypes.c_void_p))
    return out


def threads() -> int:
    return int(load().oracle_default_threads())


# ---- (1) C restatement of the reference pipeline --------------------------------------

def port_csr_binary(op, rows, pa, ca, va, pb, cb, vb, nthreads=0, timing=None):
    """op in {"add", "mul"}: returns (pos int32, crd int32, val float32).  If `timing` is a
    dict, timing["seconds"] receives the duration of the C call alone."""
    import time

    lib = load()
    keep = [_as(pa, np.int32), _as(ca, np.int32), _as(va, np.float32),
            _as(pb, np.int32), _as(cb, np.int32), _as(vb, np.float32)]
    opos, ocrd, oval, onnz = _i32p(), _i32p(), _f32p(), ctypes.c_int()
    t0 = time.perf_counter()
    rc = lib.oracle_csr_binary(
        1 if op == "mul" else 0, int(rows),
        _ptr(keep[0], ctypes.c_int32), _ptr(keep[1], ctypes.c_int32),
        _ptr(keep[2], ctypes.c_float), int(len(ca)),
        _ptr(keep[3], ctypes.c_int32), _ptr(keep[4], ctypes.c_int32),
        _ptr(keep[5], ctypes.c_float), int(len(cb)), int(nthreads),
        ctypes.byref(opos), ctypes.byref(ocrd), ctypes.byref(oval), ctypes.byref(onnz))
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_csr_binary failed ({rc})")
    n = onnz.value
    return (_take(opos, rows + 1, np.int32), _take(ocrd, n, np.int32),
            _take(oval, n, np.float32))


def port_coo_binary(op, a_crd, va, b_crd, vb, nthreads=0, timing=None):
    """a_crd / b_crd: tuple of 2 or 3 int arrays (lexicographically sorted, distinct).  If
    `timing` is a dict, timing["seconds"] receives the duration of the C call alone."""
    import time

    lib = load()
    arity = len(a_crd)
    a = [_as(x, np.int32) for x in a_crd]
    b = [_as(x, np.int32) for x in b_crd]
    fa, fb = _as(va, np.float32), _as(vb, np.float32)
    arr_t = _i32p * 3
    ap = arr_t(*[_ptr(x, ctypes.c_int32) for x in a] + [None] * (3 - arity))
    bp = arr_t(*[_ptr(x, ctypes.c_int32) for x in b] + [None] * (3 - arity))
    out = arr_t()
    oval, onnz = _f32p(), ctypes.c_int()
    t0 = time.perf_counter()
    rc = lib.oracle_coo_binary(1 if op == "mul" else 0, arity, ap, _ptr(fa, ctypes.c_float),
                               int(len(va)), bp, _ptr(fb, ctypes.c_float), int(len(vb)),
                               int(nthreads), out, ctypes.byref(oval), ctypes.byref(onnz))
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_coo_binary failed ({rc})")
    n = onnz.value
    crd = tuple(_take(out[d], n, np.int32) for d in range(arity))
    return crd, _take(oval, n, np.float32)


def port_csf3_union(a_levels, a_val, b_levels, b_val, timing=None, nthreads=None):
    """levels = (crd_i, pos_j, crd_j, pos_k, crd_k).  Returns (levels, val).  If `timing` is
    a dict, timing["seconds"] receives the duration of the C call alone.  nthreads=None runs
    the serial lattice (oracle_csf3_union); a count (0 = all cores) runs the range-parallel
    restatement (oracle_csf3_union_mt), whose result is the same."""
    import time

    lib = load()

    def prep(levels, val):
        ci, pj, cj, pk, ck = (_as(x, np.int32) for x in levels)
        v = _as(val, np.float32)
        return (ci, len(levels[0]), pj, cj, len(levels[2]), pk, ck, v, len(levels[4]))

    pa, pb = prep(a_levels, a_val), prep(b_levels, b_val)

    def args(p):
        ci, ni, pj, cj, nj, pk, ck, v, nk = p
        return [_ptr(ci, ctypes.c_int32), ni, _ptr(pj, ctypes.c_int32), _ptr(cj, ctypes.c_int32),
                nj, _ptr(pk, ctypes.c_int32), _ptr(ck, ctypes.c_int32), _ptr(v, ctypes.c_float),
                nk]

    outs = [_i32p() for _ in range(5)]
    oval = _f32p()
    ns = [ctypes.c_int() for _ in range(3)]
    t0 = time.perf_counter()
    if nthreads is None:
        rc = lib.oracle_csf3_union(*args(pa), *args(pb), *[ctypes.byref(o) for o in outs],
                                   ctypes.byref(oval), *[ctypes.byref(n) for n in ns])
    else:
        rc = lib.oracle_csf3_union_mt(*args(pa), *args(pb), int(nthreads),
                                      *[ctypes.byref(o) for o in outs], ctypes.byref(oval),
                                      *[ctypes.byref(n) for n in ns])
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_csf3_union failed ({rc})")
    ni, nj, nk = (n.value for n in ns)
    levels = (_take(outs[0], ni, np.int32), _take(outs[1], ni + 1, np.int32),
              _take(outs[2], nj, np.int32), _take(outs[3], nj + 1, np.int32),
              _take(outs[4], nk, np.int32))
    return levels, _take(oval, nk, np.float32)


def port_csr_add3(rows, a, b, c, timing=None, nthreads=None):
    """a, b, c = (pos, crd, val).  Returns (pos int32, crd int32, val float32).  If `timing`
    is a dict, timing["seconds"] receives the duration of the C call alone.  nthreads=None
    runs the serial lattice; a count (0 = all cores) the row-range-parallel restatement."""
    import time

    lib = load()
    keep = []
    for t in (a, b, c):
        keep += [_as(t[0], np.int32), _as(t[1], np.int32), _as(t[2], np.float32)]
    args = []
    for i in range(0, 9, 3):
        args += [_ptr(keep[i], ctypes.c_int32), _ptr(keep[i + 1], ctypes.c_int32),
                 _ptr(keep[i + 2], ctypes.c_float)]
    opos, ocrd, oval, onnz = _i32p(), _i32p(), _f32p(), ctypes.c_int()
    t0 = time.perf_counter()
    if nthreads is None:
        rc = lib.oracle_csr_add3(int(rows), *args, ctypes.byref(opos), ctypes.byref(ocrd),
                                 ctypes.byref(oval), ctypes.byref(onnz))
    else:
        rc = lib.oracle_csr_add3_mt(int(rows), *args, int(nthreads), ctypes.byref(opos),
                                    ctypes.byref(ocrd), ctypes.byref(oval), ctypes.byref(onnz))
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_csr_add3 failed ({rc})")
    n = onnz.value
    return (_take(opos, rows + 1, np.int32), _take(ocrd, n, np.int32),
            _take(oval, n, np.float32))


def port_dcsr_binary(op, a_levels, a_val, b_levels, b_val, timing=None, nthreads=None):
    """levels = (crd_i, pos_j, crd_j).  op = "add" | "mul".  Returns (levels, val).  If
    `timing` is a dict, timing["seconds"] receives the duration of the C call alone.
    nthreads=None runs the serial lattice; a count (0 = all cores) the range-parallel
    restatement."""
    import time

    lib = load()
    ka = [_as(x, np.int32) for x in a_levels] + [_as(a_val, np.float32), len(a_levels[0])]
    kb = [_as(x, np.int32) for x in b_levels] + [_as(b_val, np.float32), len(b_levels[0])]

    def args(k):
        ci, pj, cj, v, ni = k
        return [_ptr(ci, ctypes.c_int32), ni, _ptr(pj, ctypes.c_int32),
                _ptr(cj, ctypes.c_int32), _ptr(v, ctypes.c_float)]

    outs = [_i32p() for _ in range(3)]
    oval = _f32p()
    ni, nj = ctypes.c_int(), ctypes.c_int()
    t0 = time.perf_counter()
    if nthreads is None:
        rc = lib.oracle_dcsr_binary(1 if op == "mul" else 0, *args(ka), *args(kb),
                                    *[ctypes.byref(o) for o in outs], ctypes.byref(oval),
                                    ctypes.byref(ni), ctypes.byref(nj))
    else:
        rc = lib.oracle_dcsr_binary_mt(1 if op == "mul" else 0, *args(ka), *args(kb),
                                       int(nthreads), *[ctypes.byref(o) for o in outs],
                                       ctypes.byref(oval), ctypes.byref(ni), ctypes.byref(nj))
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_dcsr_binary failed ({rc})")
    levels = (_take(outs[0], ni.value, np.int32), _take(outs[1], ni.value + 1, np.int32),
              _take(outs[2], nj.value, np.int32))
    return levels, _take(oval, nj.value, np.float32)


def port_sssmm(rows, cols, a, b, c, row_list=None, nthreads=0, timing=None):
    """Masked SpGEMM: a, b, c = (pos, crd, val); Z has C's pattern restricted to the entries
    some product reaches.  `row_list` restricts the work to those rows.  Returns
    (pos int32, crd int32, val float32)."""
    import time

    lib = load()
    keep = []
    for t in (a, b, c):
        keep += [_as(t[0], np.int32), _as(t[1], np.int32), _as(t[2], np.float32)]
    args = []
    for i in range(0, 9, 3):
        args += [_ptr(keep[i], ctypes.c_int32), _ptr(keep[i + 1], ctypes.c_int32),
                 _ptr(keep[i + 2], ctypes.c_float)]
    rl = None if row_list is None else _as(row_list, np.int32)
    opos, ocrd, oval, onnz = _i32p(), _i32p(), _f32p(), ctypes.c_int()
    t0 = time.perf_counter()
    rc = lib.oracle_sssmm(int(rows), int(cols), *args,
                          None if rl is None else _ptr(rl, ctypes.c_int32),
                          0 if row_list is None else len(row_list), int(nthreads),
                          ctypes.byref(opos), ctypes.byref(ocrd), ctypes.byref(oval),
                          ctypes.byref(onnz))
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_sssmm failed ({rc})")
    n = onnz.value
    return (_take(opos, rows + 1, np.int32), _take(ocrd, n, np.int32),
            _take(oval, n, np.float32))


def port_spgemm(rows, inner, cols, pa, ca, va, pb, cb, vb, nthreads=0):
    """ESC semantics on the CPU: returns (pos int64, crd int32, val float32)."""
    lib = load()
    keep = [_as(pa, np.int32), _as(ca, np.int32), _as(va, np.float32),
            _as(pb, np.int32), _as(cb, np.int32), _as(vb, np.float32)]
    opos, ocrd, oval, onnz = _i64p(), _i32p(), _f32p(), ctypes.c_int64()
    rc = lib.oracle_spgemm(int(rows), int(inner), int(cols),
                           _ptr(keep[0], ctypes.c_int32), _ptr(keep[1], ctypes.c_int32),
                           _ptr(keep[2], ctypes.c_float), _ptr(keep[3], ctypes.c_int32),
                           _ptr(keep[4], ctypes.c_int32), _ptr(keep[5], ctypes.c_float),
                           int(nthreads), ctypes.byref(opos), ctypes.byref(ocrd),
                           ctypes.byref(oval), ctypes.byref(onnz))
    if rc != 0:
        raise RuntimeError(f"oracle_spgemm failed ({rc})")
    n = onnz.value
    return (_take(opos, rows + 1, np.int64), _take(ocrd, n, np.int32),
            _take(oval, n, np.float32))


# ---- (2) closed forms from the mathematics --------------------------------------------

def _rows_of(pos):
    pos = np.asarray(pos, dtype=np.int64)
    return np.repeat(np.arange(len(pos) - 1, dtype=np.int64), np.diff(pos))


def _lookup(src_keys, src_vals, keys):
    """(present mask, value where present) of sorted `keys` in sorted `src_keys`."""
    if len(src_keys) == 0:
        return np.zeros(len(keys), bool), np.zeros(len(keys), np.float32)
    idx = np.searchsorted(src_keys, keys)
    idx_c = np.minimum(idx, len(src_keys) - 1)
    hit = (idx < len(src_keys)) & (src_keys[idx_c] == keys)
    return hit, np.where(hit, src_vals[idx_c], np.float32(0)).astype(np.float32)


def _combine_keys(op, ka, va, kb, vb):
    """Sorted result keys and f32 values of the union (add) / intersection (mul)."""
    va = np.asarray(va, np.float32)
    vb = np.asarray(vb, np.float32)
    keys = np.union1d(ka, kb) if op == "add" else np.intersect1d(ka, kb, assume_unique=True)
    hit_a, xa = _lookup(ka, va, keys)
    hit_b, xb = _lookup(kb, vb, keys)
    both = hit_a & hit_b
    if op == "add":
        val = np.where(both, xa + xb, np.where(hit_a, xa, xb))  # one f32 add or a copy
    else:
        val = xa * xb  # one f32 multiply
    return keys, val.astype(np.float32)


def closed_csr_binary(op, rows, cols, pa, ca, va, pb, cb, vb):
    """Union (add) or intersection (mul) of the (row, col) key sets; values by one f32 op.
    Explicit zeros are kept (no pruning)."""
    width = int(cols) + 1
    ka = _rows_of(pa) * width + np.asarray(ca, np.int64)
    kb = _rows_of(pb) * width + np.asarray(cb, np.int64)
    keys, val = _combine_keys(op, ka, va, kb, vb)
    r = keys // width
    crd = (keys % width).astype(np.int32)
    pos = np.zeros(int(rows) + 1, np.int64)
    np.add.at(pos, r + 1, 1)
    return np.cumsum(pos).astype(np.int32), crd, val


def port_csf3_inner(a_levels, a_val, b_levels, b_val, nthreads=0, timing=None) -> float:
    """Inner product of two CSF3 tensors (levels = (crd_i, pos_j, crd_j, pos_k, crd_k)) as
    the float64 sum of the float32 products (oracle_csf3_inner); nthreads 0 = all cores."""
    import time

    lib = load()

    def prep(levels, val):
        ci, pj, cj, pk, ck = (_as(x, np.int32) for x in levels)
        return ci, len(levels[0]), pj, cj, pk, ck, _as(val, np.float32)

    def args(p):
        ci, ni, pj, cj, pk, ck, v = p
        return [_ptr(ci, ctypes.c_int32), ni, _ptr(pj, ctypes.c_int32),
                _ptr(cj, ctypes.c_int32), _ptr(pk, ctypes.c_int32), _ptr(ck, ctypes.c_int32),
                _ptr(v, ctypes.c_float)]

    pa, pb = prep(a_levels, a_val), prep(b_levels, b_val)
    out = ctypes.c_double()
    t0 = time.perf_counter()
    rc = lib.oracle_csf3_inner(*args(pa), *args(pb), int(nthreads), ctypes.byref(out))
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_csf3_inner failed ({rc})")
    return out.value


def port_coo3_inner(a_crd, va, b_crd, vb, nthreads=0, timing=None) -> float:
    """Inner product of two COO3 tensors (crd = (i, j, k) arrays sorted lexicographically,
    no duplicates) as the float64 sum of the float32 products (oracle_coo3_inner)."""
    import time

    lib = load()
    a = [_as(x, np.int32) for x in a_crd] + [_as(va, np.float32), len(va)]
    b = [_as(x, np.int32) for x in b_crd] + [_as(vb, np.float32), len(vb)]

    def args(p):
        return [_ptr(p[0], ctypes.c_int32), _ptr(p[1], ctypes.c_int32),
                _ptr(p[2], ctypes.c_int32), _ptr(p[3], ctypes.c_float), p[4]]

    out = ctypes.c_double()
    t0 = time.perf_counter()
    rc = lib.oracle_coo3_inner(*args(a), *args(b), int(nthreads), ctypes.byref(out))
    if timing is not None:
        timing["seconds"] = time.perf_counter() - t0
    if rc != 0:
        raise RuntimeError(f"oracle_coo3_inner failed ({rc})")
    return out.value


def closed_inner(shape, a_crd, va, b_crd, vb) -> float:
    """Inner product from the mathematics: the coordinate tuples both hold (packed keys,
    np.intersect1d), their float32 products summed in float64."""
    ka, kb = _tuple_keys(a_crd, shape), _tuple_keys(b_crd, shape)
    _, ia, ib = np.intersect1d(ka, kb, assume_unique=True, return_indices=True)
    prod = np.asarray(va, np.float32)[ia] * np.asarray(vb, np.float32)[ib]
    return float(np.sum(prod.astype(np.float64)))


def _tuple_keys(crd, shape):
    k = np.zeros(len(crd[0]), dtype=np.int64)
    for c, n in zip(crd, shape):
        k = k * (int(n) + 1) + np.asarray(c, np.int64)
    return k


def closed_coo_binary(op, shape, a_crd, va, b_crd, vb):
    """Union / intersection of coordinate tuples (keys packed in int64; shape must allow)."""
    bits = sum(int(np.ceil(np.log2(int(n) + 2))) for n in shape)
    if bits > 62:
        raise ValueError("shape too large for packed keys")
    keys, val = _combine_keys(op, _tuple_keys(a_crd, shape), va, _tuple_keys(b_crd, shape), vb)
    crd = []
    rest = keys.copy()
    for n in reversed(shape):
        crd.append((rest % (int(n) + 1)).astype(np.int32))
        rest //= (int(n) + 1)
    return tuple(reversed(crd)), val


def closed_csr_add3(rows, cols, a, b, c):
    """Union of the three (row, col) key sets; each value the sum of the present operands
    in the order (a + b) + c, in float32."""
    width = int(cols) + 1
    keys_of = [(_rows_of(t[0]) * width + np.asarray(t[1], np.int64)) for t in (a, b, c)]
    keys = np.union1d(np.union1d(keys_of[0], keys_of[1]), keys_of[2])
    hits = [_lookup(k, np.asarray(t[2], np.float32), keys) for k, t in zip(keys_of, (a, b, c))]
    (ha, xa), (hb, xb), (hc, xc) = hits
    ab = np.where(ha & hb, xa + xb, np.where(ha, xa, xb)).astype(np.float32)
    val = np.where(ha | hb, np.where(hc, ab + xc, ab), xc).astype(np.float32)
    pos = np.zeros(int(rows) + 1, np.int64)
    np.add.at(pos, keys // width + 1, 1)
    return np.cumsum(pos).astype(np.int32), (keys % width).astype(np.int32), val


def closed_sssmm_f64(rows, inner, cols, a, b, c):
    """Masked product from scipy: structure = pattern(A) pattern(B) intersected with
    pattern(C) (0/1 patterns, so cancellation keeps entries); values c_ik * (A B)_ik in
    float64."""
    import scipy.sparse as sp

    def mat(t, shape, ones=False):
        v = np.ones(len(t[1])) if ones else np.asarray(t[2], np.float64)
        return sp.csr_matrix((v, np.asarray(t[1]), np.asarray(t[0])), shape=shape)

    pat = (mat(a, (rows, inner), True) @ mat(b, (inner, cols), True)).tocsr()
    cpat = mat(c, (rows, cols), True)
    keep = pat.multiply(cpat).tocsr()
    keep.eliminate_zeros()
    keep.sort_indices()
    prod = (mat(a, (rows, inner)) @ mat(b, (inner, cols))).multiply(mat(c, (rows, cols)))
    prod = sp.csr_matrix(prod)
    width = cols + 1
    kk = _rows_of(keep.indptr) * width + keep.indices
    prod.sort_indices()
    kp = _rows_of(prod.indptr) * width + prod.indices
    vals = np.zeros(keep.nnz, np.float64)
    hit, v = _lookup(kp, prod.data, kk) if len(kp) else (np.zeros(keep.nnz, bool), vals)
    vals[hit] = np.asarray(prod.data, np.float64)[np.searchsorted(kp, kk[hit])]
    return keep.indptr.astype(np.int32), keep.indices.astype(np.int32), vals


def closed_dcsr_binary(op, rows, cols, a_levels, a_val, b_levels, b_val):
    """DCSR result from the mathematics: the stored row ids are the union (add) or the
    intersection (mul) of the operands' row ids; each row's entries are the CSR union /
    intersection of the expanded matrices (closed_csr_binary)."""
    def expand(levels):
        ci, pj, _ = (np.asarray(x, np.int64) for x in levels)
        pos = np.zeros(int(rows) + 1, np.int64)
        pos[ci + 1] = np.diff(pj)
        return np.cumsum(pos)

    pos, crd, val = closed_csr_binary(op, rows, cols, expand(a_levels), a_levels[2], a_val,
                                      expand(b_levels), b_levels[2], b_val)
    ra, rb = np.asarray(a_levels[0], np.int64), np.asarray(b_levels[0], np.int64)
    ids = np.union1d(ra, rb) if op == "add" else np.intersect1d(ra, rb)
    pos = np.asarray(pos, np.int64)
    pj = np.append(pos[ids], pos[-1]) if len(ids) else np.array([pos[-1]], np.int64)
    return (ids.astype(np.int32), pj.astype(np.int32), crd), val


def closed_spgemm_f64(rows, inner, cols, pa, ca, va, pb, cb, vb):
    """C = A B in float64 from f32 products (scipy), structure without pruning."""
    import scipy.sparse as sp

    a = sp.csr_matrix((np.asarray(va, np.float64), np.asarray(ca), np.asarray(pa)),
                      shape=(rows, inner))
    b = sp.csr_matrix((np.asarray(vb, np.float64), np.asarray(cb), np.asarray(pb)),
                      shape=(inner, cols))
    # pattern product (ones) gives the exact structure even where values cancel
    pat = (sp.csr_matrix((np.ones(len(ca)), np.asarray(ca), np.asarray(pa)), shape=(rows, inner))
           @ sp.csr_matrix((np.ones(len(cb)), np.asarray(cb), np.asarray(pb)),
                           shape=(inner, cols)))
    pat.sort_indices()
    c = (a @ b).tocsr()
    c.sort_indices()
    # align values onto the pattern (cancellation can drop entries from c)
    vals = np.zeros(pat.nnz, np.float64)
    pr = _rows_of(pat.indptr)
    cr = _rows_of(c.indptr)
    kp = pr * (cols + 1) + pat.indices
    kc = cr * (cols + 1) + c.indices
    vals[np.searchsorted(kp, kc)] = c.data
    return pat.indptr.astype(np.int64), pat.indices.astype(np.int32), vals
