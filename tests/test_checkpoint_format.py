"""NEURCKPT container format on the CPU (no tensors, so no device needed).

The expected bytes are assembled field by field from the layout the
reference documents (pyneural/checkpoint.py:4-35 of the reference): magic,
version, count, epoch / best_loss / lr, the optimizer header and payload, the
state-blob size.  Reading covers versions 1-3, the optimizer payload applied
to an optimizer object, the strict type check and every error the reference
raises (bad magic, unknown version, count mismatch, truncation, missing file).
"""

import struct

import pytest

from pyneural import checkpoint as ck


class SGD:  # class names select the optimizer type, as in the reference
    def __init__(self):
        self.momentum, self.lr = 0.9, 0.05


class AdamW:
    def __init__(self):
        self.beta1, self.beta2, self.epsilon, self.weight_decay, self.lr = 0.8, 0.99, 1e-7, 0.1, 1e-3


def _v3_bytes(epoch, best, lr, has, typ, payload, blob=b"", ntensors=0):
    return (b"NEURCKPT" + struct.pack("<II", 3, ntensors) + struct.pack("<I", epoch) + struct.pack("<d", best)
            + struct.pack("<d", lr) + struct.pack("<BBH", has, typ, 0) + struct.pack("<ddddd", *payload)
            + struct.pack("<Q", len(blob)) + blob)


def test_save_layout_without_optimizer(tmp_path):
    p = tmp_path / "a.ckpt"
    ck.save_checkpoint(p, [], None, epoch=7, best_loss=0.5, lr=0.01)
    assert p.read_bytes() == _v3_bytes(7, 0.5, 0.01, 0, 0, (0.0,) * 5)
    info = ck.load_checkpoint(p, [])
    assert info == {"epoch": 7, "best_loss": 0.5, "lr": 0.01, "optimizer_type": 0}


def test_save_layout_optimizer_payload(tmp_path):
    p = tmp_path / "b.ckpt"
    ck.save_checkpoint(p, [], AdamW(), epoch=3, lr=2e-3)
    assert p.read_bytes() == _v3_bytes(3, float("inf"), 2e-3, 1, 3, (0.0, 0.8, 0.99, 1e-7, 0.1))
    ck.save_checkpoint(p, [], SGD(), epoch=1)
    assert p.read_bytes() == _v3_bytes(1, float("inf"), 0.0, 1, 1, (0.9, 0.0, 0.0, 0.0, 0.0))


def test_load_applies_payload_and_lr(tmp_path):
    p = tmp_path / "c.ckpt"
    p.write_bytes(_v3_bytes(11, 0.25, 0.125, 1, 3, (0.0, 0.5, 0.75, 1e-6, 0.2)))
    opt = AdamW()
    info = ck.load_checkpoint(p, [], opt)
    assert info == {"epoch": 11, "best_loss": 0.25, "lr": 0.125, "optimizer_type": 3}
    assert (opt.beta1, opt.beta2, opt.epsilon, opt.weight_decay, opt.lr) == (0.5, 0.75, 1e-6, 0.2, 0.125)
    with pytest.raises(ValueError, match="Optimizer type mismatch"):
        ck.load_checkpoint(p, [], SGD(), strict_optimizer=True)
    ck.load_checkpoint(p, [], SGD())  # not strict: accepted


def test_versions_1_and_2(tmp_path):
    p = tmp_path / "v1.ckpt"
    p.write_bytes(b"NEURCKPT" + struct.pack("<II", 1, 0) + struct.pack("<Idd", 4, 1.5, 0.3))
    assert ck.load_checkpoint(p, []) == {"epoch": 4, "best_loss": 1.5, "lr": 0.3, "optimizer_type": 0}
    p = tmp_path / "v2.ckpt"
    p.write_bytes(b"NEURCKPT" + struct.pack("<II", 2, 0) + struct.pack("<Idd", 5, 2.5, 0.4)
                  + struct.pack("<BBH", 1, 1, 0) + struct.pack("<ddddd", 0.7, 0, 0, 0, 0))
    opt = SGD()
    assert ck.load_checkpoint(p, [], opt)["optimizer_type"] == 1
    assert opt.momentum == 0.7 and opt.lr == 0.4


def test_errors(tmp_path):
    with pytest.raises(FileNotFoundError):
        ck.load_checkpoint(tmp_path / "missing.ckpt", [])
    p = tmp_path / "e.ckpt"
    p.write_bytes(b"NOTACKPT" + b"\0" * 40)
    with pytest.raises(ValueError, match="magic"):
        ck.load_checkpoint(p, [])
    p.write_bytes(b"NEURCKPT" + struct.pack("<II", 4, 0) + b"\0" * 20)
    with pytest.raises(ValueError, match="version"):
        ck.load_checkpoint(p, [])
    p.write_bytes(_v3_bytes(0, 0.0, 0.0, 0, 0, (0.0,) * 5, ntensors=2))
    with pytest.raises(ValueError, match="count mismatch"):
        ck.load_checkpoint(p, [])
    full = _v3_bytes(0, 0.0, 0.0, 1, 3, (0.0,) * 5, blob=b"x" * 100)
    p.write_bytes(full[:36])
    with pytest.raises(IOError, match="optimizer header"):
        ck.load_checkpoint(p, [])
    p.write_bytes(full[:50])
    with pytest.raises(IOError, match="optimizer payload"):
        ck.load_checkpoint(p, [])
    p.write_bytes(full[:82])
    with pytest.raises(IOError, match="blob size"):
        ck.load_checkpoint(p, [])
    p.write_bytes(full[:-1])
    with pytest.raises(IOError, match="state blob"):
        ck.load_checkpoint(p, [])


class Adam:
    """An optimizer whose state export fails (a handle the library refuses)."""

    def __init__(self):
        self.beta1, self.beta2, self.epsilon, self.weight_decay, self.lr = 0.9, 0.999, 1e-8, 0.0, 1e-3
        self._ptr = 1

    def state_bytes(self):
        from pyneural.core import NeuralException
        raise NeuralException(3, "opt_state_export failed")


def test_save_when_state_export_fails(tmp_path):
    """A failing export writes the checkpoint with an empty state blob, as the
    reference's _export_optimizer_state_blob does (checkpoint.py:99-114),
    instead of raising out of save_checkpoint."""
    p = tmp_path / "e.ckpt"
    ck.save_checkpoint(p, [], Adam(), epoch=2, best_loss=1.5, lr=1e-3)
    assert p.read_bytes() == _v3_bytes(2, 1.5, 1e-3, 1, 2, (0.0, 0.9, 0.999, 1e-8, 0.0))
    info = ck.load_checkpoint(p, [], Adam())
    assert info == {"epoch": 2, "best_loss": 1.5, "lr": 1e-3, "optimizer_type": 2}
