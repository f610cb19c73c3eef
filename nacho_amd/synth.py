"""Seeded synthetic operands for the benchmark configurations.

Every generator uses numpy.random.default_rng(seed), int32 indices and float32 values, with
coordinates sorted and distinct within every fibre.  The formulas are the ones the
benchmark configurations name (the reference's synthetic heat-map generator rescales row
lengths to a target nnz the same way, benchmarks/heatmap_csr_add.py:59-60):

  C1  csr_add 4096 x 4096: row length ~ Binomial(4096, 0.01), uniform distinct columns,
      values U[-1, 1]; seeds A = 1, B = 2.
  C2  csr_add 2^20 x 2^20: L = min(zipf(1.6), 65536), rescaled
      L = clip(round(L * 16 * 2^20 / sum(L)), 0, 65536); uniform distinct columns;
      values U[-1, 1]; seeds A = 1, B = 2.
  C3  csr_mul: A as C2 (seed 1); B keeps each entry of A's row with p = 0.5 and adds as many
      fresh uniform columns not in A's row as it dropped (seed 3).
  C4  SpGEMM A*A: R-MAT scale 20, 8 * 2^20 edge draws, (a, b, c, d) = (.57, .19, .19, .05),
      20 recursive quadrant draws, no vertex permutation, duplicates merged; values
      U[0.5, 1.5]; seed 1.
  C5  CSF3 / COO3 add: shape (200000, 100000, 1000), 20M draws each; i = zipf(1.3) with
      draws above 200000 rejected, minus 1; j, k uniform; deduplicated and sorted
      lexicographically; values U[-1, 1]; seeds A = 1, B = 2.

A CSR operand is returned as (pos int32[rows+1], crd int32[nnz], val float32[nnz]).
"""

from __future__ import annotations

import numpy as np

C2_ROWS = 1 << 20
C4_SCALE = 20
C5_SHAPE = (200_000, 100_000, 1_000)


def _distinct_columns(rng, lengths, ncols, exclude_keys=None):
    """Per-row distinct uniform columns in [0, ncols), sorted; returns (pos, crd).

    Rows are filled by drawing with replacement and keeping distinct (row, col) pairs, then
    redrawing each row's shortfall until every row holds its length.  `exclude_keys`
    (sorted int64 row*ncols+col) are never produced.
    """
    lengths = np.asarray(lengths, dtype=np.int64)
    rows = len(lengths)
    have = np.zeros(0, dtype=np.int64)
    need = lengths.copy()
    while True:
        total = int(need.sum())
        if total == 0:
            break
        r = np.repeat(np.arange(rows, dtype=np.int64), need)
        c = rng.integers(0, ncols, size=total, dtype=np.int64)
        keys = r * ncols + c
        if exclude_keys is not None and len(exclude_keys):
            keys = keys[~np.isin(keys, exclude_keys, assume_unique=False)]
        have = np.union1d(have, keys)
        counts = np.bincount(have // ncols, minlength=rows)
        need = np.maximum(lengths - counts, 0)
        if np.any(counts > lengths):  # cannot happen: draws never exceed the shortfall
            raise AssertionError("row overfilled")
    pos = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(have // ncols, minlength=rows), out=pos[1:])
    return pos.astype(np.int32), (have % ncols).astype(np.int32)


def _values(rng, n, lo=-1.0, hi=1.0):
    return rng.uniform(lo, hi, size=n).astype(np.float32)


def binomial_csr(rows, cols, p, seed):
    """C1-style operand: row length ~ Binomial(cols, p)."""
    rng = np.random.default_rng(seed)
    lengths = rng.binomial(cols, p, size=rows)
    pos, crd = _distinct_columns(rng, lengths, cols)
    return pos, crd, _values(rng, len(crd))


def c1_operands():
    return binomial_csr(4096, 4096, 0.01, 1), binomial_csr(4096, 4096, 0.01, 2)


def zipf_lengths(rng, rows, alpha=1.6, cap=65536, mean=16):
    raw = np.minimum(rng.zipf(alpha, size=rows), cap).astype(np.float64)
    scaled = np.rint(raw * (mean * rows) / raw.sum())
    return np.clip(scaled, 0, cap).astype(np.int64)


def zipf_csr(rows, seed, alpha=1.6, cap=65536, mean=16, cols=None):
    """C2-style operand: rescaled capped Zipf row lengths, uniform distinct columns."""
    cols = rows if cols is None else cols
    rng = np.random.default_rng(seed)
    lengths = zipf_lengths(rng, rows, alpha, cap, mean)
    pos, crd = _distinct_columns(rng, lengths, cols)
    return pos, crd, _values(rng, len(crd))


def c2_operands(rows=C2_ROWS):
    return zipf_csr(rows, 1), zipf_csr(rows, 2)


def overlap_partner(a, cols, seed, keep=0.5):
    """C3's B: keep each entry of A with probability `keep`, add as many fresh columns."""
    pos, crd, _ = a
    rng = np.random.default_rng(seed)
    rows = len(pos) - 1
    row_of = np.repeat(np.arange(rows, dtype=np.int64), np.diff(pos.astype(np.int64)))
    a_keys = row_of * cols + crd
    kept = rng.random(len(crd)) < keep
    kept_keys = a_keys[kept]
    dropped = np.bincount(row_of[~kept], minlength=rows)
    _, fresh = _distinct_columns(rng, dropped, cols, exclude_keys=a_keys)
    fresh_rows = np.repeat(np.arange(rows, dtype=np.int64), dropped)
    keys = np.union1d(kept_keys, fresh_rows * cols + fresh)
    b_pos = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(keys // cols, minlength=rows), out=b_pos[1:])
    return b_pos.astype(np.int32), (keys % cols).astype(np.int32), _values(rng, len(keys))


def c3_operands(rows=C2_ROWS):
    a = zipf_csr(rows, 1)
    return a, overlap_partner(a, rows, 3)


def rmat_csr(scale, edge_factor=8, probs=(0.57, 0.19, 0.19, 0.05), seed=1,
             values=(0.5, 1.5)):
    """R-MAT graph adjacency as CSR (C4 operand).  No vertex permutation."""
    rng = np.random.default_rng(seed)
    n = 1 << scale
    edges = edge_factor * n
    a, b, c, _ = probs
    row = np.zeros(edges, dtype=np.int64)
    col = np.zeros(edges, dtype=np.int64)
    for _level in range(scale):
        r = rng.random(edges)
        down = r >= a + b                       # quadrants c, d
        right = ((r >= a) & (r < a + b)) | (r >= a + b + c)  # quadrants b, d
        row = (row << 1) | down
        col = (col << 1) | right
    keys = np.unique(row * n + col)
    pos = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(np.bincount(keys // n, minlength=n), out=pos[1:])
    return (pos.astype(np.int32), (keys % n).astype(np.int32),
            _values(rng, len(keys), values[0], values[1]))


def c4_operand(scale=C4_SCALE):
    return rmat_csr(scale)


def zipf3_coords(n_draws, shape, seed, alpha=1.3):
    """C5 operand: sorted distinct (i, j, k) rows and their values."""
    rng = np.random.default_rng(seed)
    si, sj, sk = shape
    i = np.zeros(0, dtype=np.int64)
    while len(i) < n_draws:
        draw = rng.zipf(alpha, size=n_draws - len(i))
        i = np.concatenate([i, draw[draw <= si] - 1])
    j = rng.integers(0, sj, size=n_draws, dtype=np.int64)
    k = rng.integers(0, sk, size=n_draws, dtype=np.int64)
    keys = np.unique((i * sj + j) * sk + k)
    coords = np.stack([keys // (sj * sk), (keys // sk) % sj, keys % sk], axis=1).astype(np.int32)
    return coords, _values(rng, len(keys))


def c5_operands(n_draws=20_000_000, shape=C5_SHAPE):
    return zipf3_coords(n_draws, shape, 1), zipf3_coords(n_draws, shape, 2)


def csr_bytes(rows, nnz_a, nnz_b, nnz_c):
    """Algorithmic bytes of a CSR add/mul: every array of A, B and C once."""
    return 3 * 4 * (rows + 1) + 8 * (nnz_a + nnz_b + nnz_c)
