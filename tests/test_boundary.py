"""The Python boundary refuses caller buffers the kernels would write or read out of
bounds, on the CPU (no kernel runs).

The C ABI takes raw device pointers with no byte counts (as the reference's kernels take
bare pointers, designs/gemv_q4/gemv_q4.h:320-328), so a y / out / h / xn / logits / ids /
vals buffer or a workspace of the wrong dtype, element count, layout or device must be
caught in q4.py before any launch: the same class of mistake as passing a bf16 activation
buffer with an f32 dtype enum, which makes the GEMV read 2 M K bytes past the buffer."""
from __future__ import annotations

import pytest
import torch


@pytest.fixture(scope="module")
def q4mod(pkg):
    import importlib
    return importlib.import_module("openflowlm-next_amd.q4")


CPU = torch.device("cpu")


def test_buf_allocates_when_absent(q4mod):
    t = q4mod._buf(None, "y", torch.float32, (3, 64), CPU)
    assert t.shape == (3, 64) and t.dtype == torch.float32 and t.is_contiguous()


def test_buf_accepts_an_exact_buffer_of_any_shape_with_the_right_count(q4mod):
    t = torch.empty(192, dtype=torch.float32)
    assert q4mod._buf(t, "y", torch.float32, (3, 64), CPU) is t


@pytest.mark.parametrize("bad,err", [
    (lambda: torch.empty(3, 64, dtype=torch.bfloat16), TypeError),        # dtype
    (lambda: torch.empty(3, 63, dtype=torch.float32), ValueError),        # too few
    (lambda: torch.empty(3, 65, dtype=torch.float32), ValueError),        # too many
    (lambda: torch.empty(64, 3, dtype=torch.float32).t(), ValueError),    # not contiguous
    (lambda: torch.empty(3, 128, dtype=torch.float32)[:, ::2], ValueError),
    (lambda: [0.0] * 192, TypeError),                                     # not a tensor
])
def test_buf_refuses(q4mod, bad, err):
    with pytest.raises(err):
        q4mod._buf(bad(), "y", torch.float32, (3, 64), CPU)


def test_buf_refuses_another_device(q4mod):
    with pytest.raises(ValueError, match="must be on"):
        q4mod._buf(torch.empty(3, 64), "y", torch.float32, (3, 64), torch.device("cuda", 0))


def test_workspace_checks(q4mod):
    ws = torch.empty(1024, dtype=torch.uint8)
    assert q4mod._ws_arg(CPU, 1024, "t", ws) == (ws.data_ptr(), 1024)
    assert q4mod._ws_arg(CPU, 512, "t", torch.empty(256, dtype=torch.float32))[1] == 1024
    with pytest.raises(ValueError, match="bytes"):
        q4mod._ws_arg(CPU, 2048, "t", ws)
    with pytest.raises(ValueError, match="contiguous"):
        q4mod._ws_arg(CPU, 16, "t", torch.empty(64, 2, dtype=torch.uint8).t())
    with pytest.raises(ValueError, match="on cuda"):
        q4mod._ws_arg(torch.device("cuda", 0), 16, "t", ws)
    with pytest.raises(TypeError):
        q4mod._ws_arg(CPU, 16, "t", bytearray(64))


def test_x_dtype_comes_from_the_tensor(q4mod):
    """The activation dtype enum is derived from the tensor, never passed separately."""
    assert q4mod._x_dtype(torch.empty(1, dtype=torch.bfloat16)) == q4mod.Q4MI_BF16
    assert q4mod._x_dtype(torch.empty(1, dtype=torch.float32)) == q4mod.Q4MI_F32
    with pytest.raises(TypeError):
        q4mod._x_dtype(torch.empty(1, dtype=torch.float16))
