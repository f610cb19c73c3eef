"""GPU parity of csr_add / csr_mul (gfx950 kernels through the C ABI) against the oracle.

Bar: pos, crd and values bit-exact (values are one IEEE binary32 add or multiply, or a
copy).  Small and medium cases compare with the C restatement of the reference pipeline and
the numpy closed form; the full 2^20 x 2^20 Zipf configs compare with the C restatement
(multi-threaded) and check size-independent invariants.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import (assert_csr_equal, check_csr_invariants, csr_from_rows,
                           random_csr)

pytestmark = pytest.mark.gpu


def to_gpu(t, rows, cols, device):
    import nacho_amd

    pos, crd, val = t
    return nacho_amd.CSR_gpu(torch.from_numpy(np.asarray(pos, np.int32)).to(device),
                             torch.from_numpy(np.asarray(crd, np.int32)).to(device),
                             torch.from_numpy(np.asarray(val, np.float32)).to(device),
                             torch.tensor([rows, cols], dtype=torch.int32))


def from_gpu(z):
    torch.cuda.synchronize()
    return (z.dim_j_offsets.cpu().numpy(), z.dim_j_indices.cpu().numpy(),
            z.values.cpu().numpy())


def gpu_op(op, a, b, rows, cols, device):
    import nacho_amd

    fn = nacho_amd.gpu_csr_add_f32 if op == "add" else nacho_amd.gpu_csr_mul_f32
    print(f"[gpu] csr_{op} rows={rows} cols={cols} nnz=({len(a[1])},{len(b[1])})", flush=True)
    z = fn(to_gpu(a, rows, cols, device), to_gpu(b, rows, cols, device))
    assert tuple(z.shape.tolist()) == (rows, cols)
    return from_gpu(z)


@pytest.mark.parametrize("op", ["add", "mul"])
def test_reference_smoke_case(gpu, op):
    rng = np.random.default_rng(0)
    a, b = random_csr(rng, 200, 180, 0.05), random_csr(rng, 200, 180, 0.05)
    got = gpu_op(op, a, b, 200, 180, gpu)
    assert_csr_equal(got, oracle.port_csr_binary(op, 200, *a, *b), "smoke")


@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("seed", range(8))
def test_random_sizes(gpu, op, seed):
    rng = np.random.default_rng(100 + seed)
    rows = int(rng.choice([1, 7, 300, 5000, 40000]))
    cols = int(rng.choice([1, 50, 3000, 100000]))
    density = float(rng.choice([0.0005, 0.003, 0.02, 0.2]))
    density = min(density, 2e6 / max(rows * cols, 1))
    a, b = random_csr(rng, rows, cols, density), random_csr(rng, rows, cols, density)
    got = gpu_op(op, a, b, rows, cols, gpu)
    want = oracle.closed_csr_binary(op, rows, cols, *a, *b)
    assert_csr_equal(got, want, f"seed={seed}")
    check_csr_invariants(got[0], got[1], rows, cols)


EDGE = {
    "both_empty": (4, 5, [[], [], [], []], [[], [], [], []]),
    "a_empty": (3, 6, [[], [], []], [[0, 5], [], [2]]),
    "no_rows": (0, 4, [], []),
    "single_entry": (1, 1, [[0]], [[0]]),
    "all_overlap": (3, 8, [[0, 3, 7], [1], [2, 4]], [[0, 3, 7], [1], [2, 4]]),
    "no_overlap": (2, 8, [[0, 2, 4, 6], [1]], [[1, 3, 5, 7], [0]]),
    "row_longer_than_tile": (2, 50000, [list(range(0, 50000, 2)), []],
                             [list(range(0, 50000, 3)), [5]]),
    "identical_long_row": (1, 9000, [list(range(9000))], [list(range(9000))]),
    "many_empty_rows": (20000, 10, [[] for _ in range(19999)] + [[1, 2]],
                        [[3]] + [[] for _ in range(19999)]),
}


@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("name", sorted(EDGE))
def test_edge_cases(gpu, op, name):
    rows, cols, ra, rb = EDGE[name]
    a, b = csr_from_rows(rows, cols, ra), csr_from_rows(rows, cols, rb)
    got = gpu_op(op, a, b, rows, cols, gpu)
    assert_csr_equal(got, oracle.closed_csr_binary(op, rows, cols, *a, *b), name)


def test_explicit_zeros_kept(gpu):
    a = csr_from_rows(2, 5, [[0, 3], [4]], [1.5, -2.0, 0.25])
    b = csr_from_rows(2, 5, [[0, 3], [4]], [-1.5, 2.0, -0.25])
    pos, crd, val = gpu_op("add", a, b, 2, 5, gpu)
    assert list(crd) == [0, 3, 4] and not val.any() and list(pos) == [0, 2, 3]


def test_mul_empty_result_early_exit(gpu):
    """Disjoint operands: zeroed offsets, empty coordinate/value arrays."""
    a = csr_from_rows(3, 10, [[0, 2], [4], []], None)
    b = csr_from_rows(3, 10, [[1, 3], [5], [9]], None)
    pos, crd, val = gpu_op("mul", a, b, 3, 10, gpu)
    assert list(pos) == [0, 0, 0, 0] and len(crd) == 0 and len(val) == 0


def test_c1_config(gpu):
    from nacho_amd import synth

    a, b = synth.c1_operands()
    got = gpu_op("add", a, b, 4096, 4096, gpu)
    assert_csr_equal(got, oracle.port_csr_binary("add", 4096, *a, *b), "C1")


@pytest.mark.parametrize("op,partner", [("add", "independent"), ("mul", "overlap"),
                                        ("add", "overlap")])
def test_zipf_medium(gpu, op, partner):
    """Zipf rows (2^15): a union of independent operands (sparse overlap: the count searches
    the pairs), an intersection, and a union of operands sharing half their entries (dense
    overlap: the count walks the tiles, each counting workgroup finding its own splits)."""
    from nacho_amd import synth

    rows = 1 << 15
    a = synth.zipf_csr(rows, 11)
    b = synth.zipf_csr(rows, 12) if partner == "independent" else \
        synth.overlap_partner(a, rows, 13)
    got = gpu_op(op, a, b, rows, rows, gpu)
    assert_csr_equal(got, oracle.closed_csr_binary(op, rows, rows, *a, *b),
                     f"zipf 2^15 {op} {partner}")


@pytest.mark.parametrize("dense_rows", [1024, 96])
def test_add_sparse_overlap_with_a_dense_block(gpu, dense_rows):
    """Union whose overlap is sparse overall (the count searches the smaller side of each row
    present in both operands) except for a block of rows where both operands hold the same
    64 columns: 1024 such rows (a whole row-pass workgroup dense in pairs) or 96.
    Bit-exact against the oracle."""
    from nacho_amd import synth

    rows, cols = 200_000, 1 << 20
    a = synth.zipf_csr(rows, 21, cols=cols)
    b = synth.zipf_csr(rows, 22, cols=cols)
    rng = np.random.default_rng(23)

    def with_dense(t, seed_cols):
        pos, crd, val = t
        lengths = np.diff(pos.astype(np.int64))
        row_cols = [crd[pos[r]:pos[r + 1]] for r in range(rows)]
        for r in range(4096, 4096 + dense_rows):
            row_cols[r] = seed_cols
            lengths[r] = len(seed_cols)
        new_pos = np.zeros(rows + 1, np.int64)
        np.cumsum(lengths, out=new_pos[1:])
        new_crd = np.concatenate(row_cols).astype(np.int32)
        new_val = rng.uniform(-1, 1, len(new_crd)).astype(np.float32)
        return new_pos.astype(np.int32), new_crd, new_val

    shared = np.sort(rng.choice(cols, 64, replace=False)).astype(np.int32)
    a, b = with_dense(a, shared), with_dense(b, shared)
    got = gpu_op("add", a, b, rows, cols, gpu)
    assert_csr_equal(got, oracle.closed_csr_binary("add", rows, cols, *a, *b),
                     f"dense block of {dense_rows} rows")


@pytest.mark.parametrize("rows", [1 << 16, 3 * 1024 + 77])
def test_add_one_entry_against_twenty(gpu, rows):
    """Union where every row of A holds one entry and every row of B twenty, half of them
    holding A's column: the count searches one entry per row, so every row-pass workgroup
    holds a record per row (1024, more than one slice's worth), and each slice's records
    are found by narrowing rounds before they are staged.  Bit-exact against the oracle."""
    rng = np.random.default_rng(31)
    cols = 1 << 20
    a_crd = rng.integers(0, cols, rows).astype(np.int32)
    b_rows = []
    for r in range(rows):
        others = rng.choice(cols, 24, replace=False)
        others = others[others != a_crd[r]][:19 if r % 2 == 0 else 20]
        row = np.concatenate([others, [a_crd[r]]]) if r % 2 == 0 else others
        b_rows.append(np.sort(row).astype(np.int32))
    a = (np.arange(rows + 1, dtype=np.int32), a_crd,
         rng.uniform(-1, 1, rows).astype(np.float32))
    b_pos = np.zeros(rows + 1, np.int64)
    np.cumsum([len(x) for x in b_rows], out=b_pos[1:])
    b_crd = np.concatenate(b_rows)
    b = (b_pos.astype(np.int32), b_crd, rng.uniform(-1, 1, len(b_crd)).astype(np.float32))
    got = gpu_op("add", a, b, rows, cols, gpu)
    assert_csr_equal(got, oracle.closed_csr_binary("add", rows, cols, *a, *b),
                     f"one entry against twenty, {rows} rows")


def _rows_of(pos):
    return np.repeat(np.arange(len(pos) - 1), np.diff(pos.astype(np.int64)))


def _csr_from_coo(rows, r, c, v):
    order = np.lexsort((c, r))
    pos = np.zeros(rows + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=rows), out=pos[1:])
    return pos.astype(np.int32), c[order].astype(np.int32), v[order].astype(np.float32)


def _pair_free_operands(case, rows=1 << 16):
    """Union operands whose write chunks hold no pairs, or only some of them.  A's columns
    are even and B's odd (Zipf rows of C2's generator, column range doubled); 45% of the rows
    keep only A's entries and 45% only B's.  'disjoint': that alone (no pair; the count
    searches the rows holding both sides and finds none); 'planted': plus one shared column
    in every 31st row holding both sides (some chunks with pairs); 'half_equal': B's rows below
    rows / 2 are A's columns (pairs in half the entries, so the count walks the tiles and
    counts outputs, and the chunks of the upper half have none)."""
    from nacho_amd import synth

    rng = np.random.default_rng(41)
    a = synth.zipf_csr(rows, 42)
    b = synth.zipf_csr(rows, 43)
    side = rng.choice(3, rows, p=[0.45, 0.45, 0.10])  # 0: A only, 1: B only, 2: both
    ra, rb = _rows_of(a[0]), _rows_of(b[0])
    ka, kb = side[ra] != 1, side[rb] != 0
    ar, ac, av = ra[ka], 2 * a[1][ka].astype(np.int64), a[2][ka]
    br, bc, bv = rb[kb], 2 * b[1][kb].astype(np.int64) + 1, b[2][kb]
    if case == "planted":
        a_first = {}
        for r_, c_ in zip(ar[::-1], ac[::-1]):
            a_first[r_] = c_
        planted = [r_ for r_ in range(0, rows, 31) if side[r_] == 2 and r_ in a_first
                   and np.any(br == r_)]
        assert planted
        br = np.concatenate([br, planted])
        bc = np.concatenate([bc, [a_first[r_] for r_ in planted]])
        bv = np.concatenate([bv, rng.uniform(-1, 1, len(planted)).astype(np.float32)])
    elif case == "half_equal":
        low_a, low_b = ar < rows // 2, br < rows // 2
        br = np.concatenate([br[~low_b], ar[low_a]])
        bc = np.concatenate([bc[~low_b], ac[low_a]])
        bv = np.concatenate([bv[~low_b], rng.uniform(-1, 1, int(low_a.sum())).astype(np.float32)])
    return _csr_from_coo(rows, ar, ac, av), _csr_from_coo(rows, br, bc, bv), 2 * rows


@pytest.mark.parametrize("case", ["disjoint", "planted", "half_equal"])
def test_add_chunks_without_pairs(gpu, case):
    """Unions whose write chunks hold no pairs (all, most, or the upper half's): the count's
    pair search finding none or a few, and the count walk over tiles half of which merge
    nothing.  Bit-exact against the numpy closed form."""
    rows = 1 << 16
    a, b, cols = _pair_free_operands(case, rows)
    print(f"[gpu] csr_add chunks without pairs case={case} nnz=({len(a[1])},{len(b[1])})",
          flush=True)
    got = gpu_op("add", a, b, rows, cols, gpu)
    assert_csr_equal(got, oracle.closed_csr_binary("add", rows, cols, *a, *b),
                     f"chunks without pairs: {case}")


def test_c2_full_size_add(gpu):
    """BASELINE C2 at full size: bit-exact against the oracle, plus invariants."""
    from nacho_amd import synth

    rows = synth.C2_ROWS
    a, b = synth.c2_operands()
    got = gpu_op("add", a, b, rows, rows, gpu)
    want = oracle.port_csr_binary("add", rows, *a, *b, nthreads=16)
    assert_csr_equal(got, want, "C2")
    check_csr_invariants(got[0], got[1], rows, rows)
    # nnz(C) = nnzA + nnzB - |A ∩ B|
    overlap = len(oracle.port_csr_binary("mul", rows, *a, *b, nthreads=16)[1])
    assert len(got[1]) == len(a[1]) + len(b[1]) - overlap


def test_c3_full_size_mul(gpu):
    from nacho_amd import synth

    rows = synth.C2_ROWS
    a, b = synth.c3_operands()
    got = gpu_op("mul", a, b, rows, rows, gpu)
    want = oracle.port_csr_binary("mul", rows, *a, *b, nthreads=16)
    assert_csr_equal(got, want, "C3")
    assert 0.45 * len(a[1]) < len(got[1]) < 0.55 * len(a[1])


def test_deterministic_and_stream(gpu):
    """Two calls, the second on a side stream, give identical bits."""
    import nacho_amd
    from nacho_amd import synth

    a = synth.zipf_csr(1 << 14, 21)
    b = synth.zipf_csr(1 << 14, 22)
    ga, gb = to_gpu(a, 1 << 14, 1 << 14, gpu), to_gpu(b, 1 << 14, 1 << 14, gpu)
    first = from_gpu(nacho_amd.gpu_csr_add_f32(ga, gb))
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        second = from_gpu(nacho_amd.gpu_csr_add_f32(ga, gb))
    assert_csr_equal(second, first, "repeat")


def test_results_are_stream_ordered(gpu):
    """A call returns once the result length is known, while its write pass may still run:
    work queued behind it on the same stream, with no host synchronisation in between, sees
    the complete result."""
    import nacho_amd
    from nacho_amd import synth

    a = synth.zipf_csr(1 << 16, 31)
    b = synth.zipf_csr(1 << 16, 32)
    want = oracle.port_csr_binary("add", 1 << 16, *a, *b, nthreads=4)
    ga, gb = to_gpu(a, 1 << 16, 1 << 16, gpu), to_gpu(b, 1 << 16, 1 << 16, gpu)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        z = nacho_amd.gpu_csr_add_f32(ga, gb)
        # queued on `side` right behind the call's kernels
        copies = [t.clone() for t in (z.dim_j_offsets, z.dim_j_indices, z.values)]
    side.synchronize()
    got = tuple(t.cpu().numpy() for t in copies)
    assert_csr_equal(got, want, "stream-ordered")


def test_concurrent_host_threads(gpu):
    """Two host threads call csr_add / csr_mul at the same time on their own streams (the
    ctypes call releases the GIL): per-thread readback words and events and the shared
    caching allocator keep every result exact."""
    import threading

    import nacho_amd
    from nacho_amd import synth

    a = synth.zipf_csr(1 << 15, 41)
    b = synth.zipf_csr(1 << 15, 42)
    want = {op: oracle.port_csr_binary(op, 1 << 15, *a, *b, nthreads=4) for op in ("add", "mul")}
    ga, gb = to_gpu(a, 1 << 15, 1 << 15, gpu), to_gpu(b, 1 << 15, 1 << 15, gpu)
    torch.cuda.synchronize(gpu)
    got, errors = {}, []

    def work(op):
        try:
            fn = nacho_amd.gpu_csr_add_f32 if op == "add" else nacho_amd.gpu_csr_mul_f32
            stream = torch.cuda.Stream(device=gpu)
            with torch.cuda.stream(stream):
                outs = [fn(ga, gb) for _ in range(6)]
                host = [from_gpu(z) for z in outs]
            got[op] = host
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=work, args=(op,)) for op in ("add", "mul")]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for op in ("add", "mul"):
        for i, z in enumerate(got[op]):
            assert_csr_equal(z, want[op], f"{op} #{i}")


def test_caller_allocator_through_c_abi(gpu):
    """Call the C entry point directly with a caller-supplied allocator (torch tensors)."""
    from nacho_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(5)
    a, b = random_csr(rng, 1000, 900, 0.01), random_csr(rng, 1000, 900, 0.01)
    ga, gb = to_gpu(a, 1000, 900, gpu), to_gpu(b, 1000, 900, gpu)
    keep = {}
    released = []

    @ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p)
    def allocate(ctx, nbytes, stream):
        t = torch.empty(int(nbytes), dtype=torch.uint8, device=gpu)
        keep[t.data_ptr()] = t
        return t.data_ptr()

    @ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)
    def release(ctx, ptr, stream):
        released.append(ptr)
        keep.pop(ptr, None)

    alloc = _lib.Allocator(None, allocate, release)

    def desc(t, rows, cols):
        return _lib.CsrDesc(rows, cols, t.dim_j_offsets.data_ptr(), t.dim_j_indices.numel(),
                            t.dim_j_indices.data_ptr(), t.values.data_ptr(), t.values.numel())

    z = _lib.CsrDesc()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    rc = lib.nacho_gpu_csr_add_f32(ctypes.byref(desc(ga, 1000, 900)),
                                   ctypes.byref(desc(gb, 1000, 900)), ctypes.byref(z), 256, 256,
                                   ctypes.c_void_p(stream), ctypes.byref(alloc))
    assert rc == 0, _lib.error_string(rc)
    torch.cuda.synchronize()
    assert len(released) >= 1  # scratch went back through the caller's allocator
    n = z.nnz

    def view(ptr, count, dtype):
        return keep[ptr].view(dtype)[:count].cpu().numpy()

    got = (view(z.dim_j_offsets, 1001, torch.int32), view(z.dim_j_indices, n, torch.int32),
           view(z.values, n, torch.float32))
    assert_csr_equal(got, oracle.closed_csr_binary("add", 1000, 900, *a, *b), "allocator")
