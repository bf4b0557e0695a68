"""mk_scatter_add_rows_noalloc — the scatter-add that allocates nothing (its
workspace is the library's fixed per-GPU scratch array) — against
mk_scatter_add_rows with a caller-supplied workspace, through the C-ABI:
bit-identical results on two calls in a row, the second smaller (the scratch
keeps the first call's contents, which must not leak into the second), both
equal to the in-order fp32 oracle; a request past the scratch size fails with
a named error before anything is launched."""

import numpy as np
import pytest
import torch

from mi355x_pjrt import kernels
from mi355x_pjrt._lib import KernelError
from oracle import native

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int32).cpu().numpy()


def test_noalloc_matches_workspace_entry_point(cuda):
    rng = np.random.default_rng(2024)
    # C4's shape first, then a smaller one: fewer rows and ids than the
    # first call left in the scratch
    for n_rows, n_ids, row_len in [(50257, 65536, 768), (997, 3001, 96)]:
        print(f"case: scatter-add noalloc rows={n_rows} ids={n_ids} row_len={row_len}", flush=True)
        table = torch.from_numpy(rng.standard_normal((n_rows, row_len)).astype(np.float32)).to(cuda)
        ids_np = rng.integers(0, n_rows, n_ids).astype(np.int32)
        ids_np[:7] = ids_np[0]  # a repeated destination
        ids = torch.from_numpy(ids_np).to(cuda)
        upd_np = rng.standard_normal((n_ids, row_len)).astype(np.float32)
        upd = torch.from_numpy(upd_np).to(cuda)
        want = kernels.scatter_add_rows(table, ids, upd)
        got = kernels.scatter_add_rows_noalloc(table, ids, upd)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(got), _bits(want))
        ref = native.scatter_add_f32(table.cpu().numpy(), ids_np, upd_np)
        np.testing.assert_array_equal(_bits(got), ref.view(np.int32))


def test_noalloc_rejects_sizes_past_the_scratch(cuda):
    n_ids = 1 << 20  # about 17 MB of sort workspace, more than the scratch holds
    table = torch.zeros(16, 4, device=cuda)
    ids = torch.zeros(n_ids, dtype=torch.int32, device=cuda)
    upd = torch.zeros(n_ids, 4, device=cuda)
    with pytest.raises(KernelError, match="scratch"):
        kernels.scatter_add_rows_noalloc(table, ids, upd)
