"""Randomised dropout call sequences (training_ops.asm:718-858).

One seeded sequence of 60 forward calls against the C library's rand()
stream: lengths 1 to 400,000 (log-uniform), a repeat of the previous call's
length and probability a third of the time (the calls whose keep bits are
made ahead), p uniform in [0, 1] or 0, 1, 1/3, on host buffers, aligned
device buffers or device buffers at a 4-byte (values) / 1-byte (mask)
offset, with a reseed now and then.  Every call's mask and output must equal
the oracle's bit for bit, and the draw counter the total length since the
last seed.
"""

import ctypes

import numpy as np

from conftest import GPU, same_bits
from test_gpu_dropout import _lib

pytestmark = GPU

CALLS = 60


def test_random_call_sequence(pn, ora):
    import torch
    lib = _lib()
    rng = np.random.default_rng(909)
    seed = 4242
    lib.neural_dropout_seed(ctypes.c_uint32(seed))
    ora.srand(seed)
    drawn = 0
    n, p = 1, 0.5
    for call in range(CALLS):
        if rng.random() < 0.08:
            seed = int(rng.integers(0, 2 ** 32))
            lib.neural_dropout_seed(ctypes.c_uint32(seed))
            ora.srand(seed)
            drawn = 0
        if call == 0 or rng.random() >= 0.33:
            n = int(np.exp(rng.uniform(0, np.log(400_000))))
            u = rng.random()
            p = float(np.float32(rng.uniform(0, 1) if u < 0.7 else [0.0, 1.0, 1.0 / 3.0][int(rng.integers(0, 3))]))
        x = rng.normal(0, 1, n + 1).astype(np.float32)
        where = int(rng.integers(0, 3))
        if where == 0:
            out, mask = np.empty(n, np.float32), np.empty(n, np.uint8)
            assert lib.neural_dropout_forward(x.ctypes.data, out.ctypes.data, mask.ctypes.data, n,
                                              ctypes.c_float(p)) == 0, (call, n, p)
            xs = x[:n]
        else:
            off = where - 1  # 0: aligned; 1: values at +4 bytes, mask at +1 byte
            xd = torch.from_numpy(x).cuda()
            od = torch.full((n + 1,), 7.0, device="cuda")
            md = torch.full((n + 4,), 9, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            assert lib.neural_dropout_forward(xd.data_ptr() + 4 * off, od.data_ptr() + 4 * off, md.data_ptr() + off,
                                              n, ctypes.c_float(p)) == 0, (call, n, p, off)
            pn.synchronize()
            out, mask = od.cpu().numpy()[off:off + n], md.cpu().numpy()[off:off + n]
            xs = x[off:off + n]
        _, wout, wmask = ora.dropout_forward(xs, p)
        same_bits(mask, wmask)
        same_bits(out, wout)
        drawn += n
        assert lib.neural_dropout_draws() == drawn, call
