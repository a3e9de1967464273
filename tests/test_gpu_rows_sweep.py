"""Randomised parity sweep of the row kernels: 36 seeded draws of rows and
columns (widths the register-resident kernel covers and widths that take the
looping kernel, partial last workgroups) for row softmax with its row max and
row sum, row sum and row max alone, and softmax cross-entropy.  Against the
fp64 oracle: row max and argmax exact, the rest rel-err <= 1e-5."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

RRED = int.from_bytes(b"RRED", "little")
ROWS = [1, 3, 64, 257, 1000]
COLS = [1, 5, 64, 100, 128, 1000, 1024, 3000, 8192]


def _draws(n=36, seed=7):
    r = np.random.default_rng(seed)
    return [(int(r.choice(ROWS)), int(r.choice(COLS)), ["softmax", "sum", "max", "xent"][int(r.integers(4))])
            for _ in range(n)]


@pytest.mark.parametrize("R,Ccols,op", _draws())
def test_row_ops_random_shapes(C, R, Ccols, op):
    r = np.random.default_rng(R * 10007 + Ccols)
    x = (2.0 * r.standard_normal((R, Ccols))).astype(np.float32)
    tx = torch.from_numpy(x).cuda()
    ry, rmx, rsx = orc.softmax_rows_f64(x)
    if op == "softmax":
        y, mx, sx = torch.empty_like(tx), torch.empty(R, device="cuda"), torch.empty(R, device="cuda")
        C.op_call(int(C.OpKind.RowSoftmax), [tx], [y, mx, sx], 0, b"", 0)
        assert orc.rel_err(y.cpu().numpy(), ry) < 1e-5
        assert np.array_equal(mx.cpu().numpy(), x.max(axis=1))
        assert orc.rel_err(sx.cpu().numpy(), rsx) < 1e-5
    elif op in ("sum", "max"):
        o = torch.empty(R, device="cuda")
        C.op_call(int(C.OpKind.RowReduce), [tx], [o], RRED, struct.pack("<i", 1 if op == "max" else 0), 0)
        if op == "max":
            assert np.array_equal(o.cpu().numpy(), x.max(axis=1))
        else:
            assert orc.rel_err(o.cpu().numpy(), rsx) < 1e-5
    else:
        lab = r.integers(0, Ccols, R).astype(np.int32)
        loss, dz = torch.empty((), device="cuda"), torch.empty_like(tx)
        am, rl = torch.empty(R, dtype=torch.int32, device="cuda"), torch.empty(R, device="cuda")
        C.op_call(int(C.OpKind.SoftmaxXent), [tx, torch.from_numpy(lab).cuda()], [loss, dz, am, rl], 0, b"", 0)
        rloss, rdz, ram, rrl = orc.softmax_xent_f64(x, lab)
        assert np.array_equal(am.cpu().numpy(), ram)
        assert abs(float(loss.item()) - rloss) <= 1e-5 * max(abs(rloss), 1e-30)
        assert orc.rel_err(dz.cpu().numpy(), rdz) < 1e-5
        assert orc.rel_err(rl.cpu().numpy(), rrl) < 1e-5
