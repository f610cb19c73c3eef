"""Real-data path on the GPU: a Matrix Market file read by parse2D, converted with to_csr
and added / multiplied on the device, against the oracle (bit-exact)."""

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("op", ["add", "mul"])
def test_mtx_file_through_csr_kernels(gpu, tmp_path, op):
    import nacho_amd
    from nacho_amd import io

    rng = np.random.default_rng(11)
    a = sp.random(3000, 3000, density=0.002, format="coo", random_state=1)
    a = sp.triu(a + a.T, format="coo")  # symmetric upper triangle; the reader mirrors it
    a.data = rng.uniform(-1, 1, a.nnz)
    f = tmp_path / "a.mtx"
    scipy.io.mmwrite(str(f), a, symmetry="symmetric")
    ta = io.parse_matrix(f, device="cpu")
    tb = (ta.to_dense() * 2.0 + torch.diag(torch.ones(3000))).to_sparse_csr()
    print(f"[gpu] mtx {op} nnz=({ta.values().numel()},{tb.values().numel()})", flush=True)
    fn = nacho_amd.gpu_csr_add_f32 if op == "add" else nacho_amd.gpu_csr_mul_f32
    z = fn(nacho_amd.to_csr(ta, gpu), nacho_amd.to_csr(tb, gpu))
    torch.cuda.synchronize()
    np_of = lambda t: (t.crow_indices().numpy().astype(np.int32),  # noqa: E731
                       t.col_indices().numpy().astype(np.int32),
                       t.values().numpy().astype(np.float32))
    pos, crd, val = oracle.port_csr_binary(op, 3000, *np_of(ta), *np_of(tb))
    np.testing.assert_array_equal(z.dim_j_offsets.cpu().numpy(), pos)
    np.testing.assert_array_equal(z.dim_j_indices.cpu().numpy(), crd)
    np.testing.assert_array_equal(z.values.cpu().numpy().view(np.int32), val.view(np.int32))
