"""The ctypes binding refuses tensors that would make the kernels read or
write out of bounds (wrong dtype, shape, layout or device) with ValueError,
before anything reaches the C-ABI.  CPU only: the checks run on host
tensors, and the MoeBlock methods are driven on an object whose library
handle is absent, so a check that let a call through would fail loudly."""
import numpy as np
import pytest
import torch

import moe_block as mb
import workloads as wl


def desc(shape=wl.C1):
    return mb.LayerDesc.of(shape)


def host(shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


def good(T=2, d=None, per_slot=False):
    d = d or desc()
    out = (T, d.n_used, d.hidden) if per_slot else (T, d.hidden)
    return (host((T, d.hidden)), host((T, d.n_used), torch.int32), host((T, d.n_used)), host(out))


def test_well_formed_host_tensors_are_refused_only_for_the_device():
    d = desc()
    for per_slot in (False, True):
        x, ids, wts, out = good(3, d, per_slot)
        with pytest.raises(ValueError, match="ROCm device"):
            mb.check_forward_args(d, x, ids, wts, out, mb.MOE_FWD_PER_SLOT if per_slot else 0)


@pytest.mark.parametrize("which, bad, msg", [
    ("x", host((2, 1024)), "shape"),                       # wrong hidden size
    ("x", host((2, 2048), torch.float16), "dtype"),
    ("x", host((2, 2048 * 2))[:, ::2], "shape|contiguous"),
    ("ids", host((2, 3), torch.int32), "shape"),           # fewer than k columns
    ("ids", host((2, 4), torch.int64), "dtype"),
    ("ids", host((3, 4), torch.int32), "shape"),           # token count differs from x
    ("wts", host((2, 4), torch.float64), "dtype"),
    ("wts", host((2, 5)), "shape"),
    ("out", host((2, 4, 2048)), "shape"),                  # per-slot out without the flag
    ("out", host((1, 2048)), "shape"),
    ("out", host((2, 2048 * 2))[:, :2048], "contiguous"),
])
def test_forward_refusals(which, bad, msg):
    d = desc()
    args = dict(zip(("x", "ids", "wts", "out"), good(2, d)))
    args[which] = bad
    with pytest.raises(ValueError, match=msg):
        mb.check_forward_args(d, args["x"], args["ids"], args["wts"], args["out"])


def test_per_slot_out_must_be_per_slot():
    d = desc()
    x, ids, wts, out = good(2, d)
    with pytest.raises(ValueError, match="shape"):
        mb.check_forward_args(d, x, ids, wts, out, mb.MOE_FWD_PER_SLOT)


def test_non_tensor_and_empty_batch():
    d = desc()
    x, ids, wts, out = good(2, d)
    with pytest.raises(ValueError, match="torch tensor"):
        mb.check_forward_args(d, np.zeros((2, 2048), np.float32), ids, wts, out)
    with pytest.raises(ValueError, match="no tokens"):
        mb.check_forward_args(d, host((0, 2048)), ids, wts, out)


def test_host_boundary_shapes():
    d = desc()
    x = np.zeros((2, 2048), np.float32)
    ids = np.zeros((2, 4), np.int32)
    wts = np.zeros((2, 4), np.float32)
    assert mb.check_host_forward_args(d, x, ids, wts) == 2
    for bx, bi, bw in [(np.zeros((2, 1024), np.float32), ids, wts), (x, np.zeros((2, 3), np.int32), wts),
                       (x, ids, np.zeros((1, 4), np.float32))]:
        with pytest.raises(ValueError, match="shape"):
            mb.check_host_forward_args(d, bx, bi, bw)


class _NoLib:
    def __getattr__(self, name):
        raise AssertionError(f"the C-ABI was reached ({name}) with arguments the wrapper should refuse")


def detached_block():
    """A MoeBlock without a device: its library calls fail the test."""
    b = mb.MoeBlock.__new__(mb.MoeBlock)
    b.lib, b.h, b.descs = _NoLib(), None, {0: desc()}
    return b


def test_methods_check_before_calling_the_library():
    b = detached_block()
    x, ids, wts, out = good(2)
    bad_x = host((2, 1024))
    calls = [
        lambda: b.forward(0, bad_x, ids, wts, out),
        lambda: b.forward_noalloc(0, bad_x, ids, wts, out),
        lambda: b.forward(0, x, host((2, 3), torch.int32), wts, out),
        lambda: b.route_forward(0, x, host((2, 16)), ids, wts, out, mode=0),       # logits of E=16, layer has 32
        lambda: b.graph_capture([0, 0], [x, x[:1]], [ids, ids[:1]], [wts, wts[:1]], [out, out[:1]]),
        lambda: b.graph_capture([0], [x], [ids], [wts], [out, out]),
        lambda: b.route(host((2, 32)), 4, 0, True, 1.0, host((2, 3), torch.int32), wts),
        lambda: b.route(host((2, 32)), 4, 0, True, 1.0, ids, wts, bias=host((31,))),
        lambda: b.group(ids, 32, host((31,), torch.int32), host((33,), torch.int32), host((8,), torch.int32)),
        lambda: b.router_logits(host((32, 1024)), x, host((2, 32))),
        lambda: b.forward_host(0, np.zeros((2, 1024), np.float32), np.zeros((2, 4), np.int32),
                               np.zeros((2, 4), np.float32)),
        lambda: b.debug_wave_sum(host((100,)), host((2,))),
    ]
    for i, c in enumerate(calls):
        with pytest.raises(ValueError):
            c()


def test_graph_capture_token_counts_must_agree():
    b = detached_block()
    x, ids, wts, out = good(2)
    with pytest.raises(ValueError):
        b.graph_capture([0, 0], [x, x[:1]], [ids, ids[:1]], [wts, wts[:1]], [out, out[:1]])
