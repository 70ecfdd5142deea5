"""``ipc_steps_noalloc`` (the static-scratch entry point) against the plan path.

Both run the same whole-step kernel with the same arithmetic; only the home
of the kernels' barrier words, f(x) buffers and exchange records differs
(the library's static device scratch against the plan's workspace), so the
states, errors and weights must agree bit for bit.  Two calls in a row per
net, the second with a smaller batch, so the second runs on the scratch the
first left behind.
"""
import ctypes

import pytest
import torch

from lich_amd import _native as nat
from lich_amd.trainer import HipIPC, IPCConfig, _ptr_array
from oracle import ipc_oracle as O
from tests.helpers import DEV, report

pytestmark = pytest.mark.gpu

T = 4
D6 = (10,) + (64,) * 6 + (784,)


def _noalloc(dims, B, x, e, w, operand, split, act, wmode, steps):
    L = len(dims) - 1
    d = (ctypes.c_int * (L + 1))(*dims)
    return nat.lib().ipc_steps_noalloc(L, d, B, _ptr_array(x), _ptr_array(e), _ptr_array(w), operand, split, act,
                                       1e-4, 0.5, wmode, steps, nat.current_stream_handle(DEV))


@pytest.mark.parametrize("dims,dtype,wmode,paths,batches", [
    (D6, torch.float16, "gemm", ("resident", "resident"), (128, 64)),
    (D6, torch.bfloat16, "gemm", ("resident", "resident"), (96, 40)),
    (D6, torch.float16, "auto", ("narrow", "narrow"), (16, 8)),
    ((10, 64, 64, 64, 784), torch.float32, "gemm", ("narrow", "resident"), (128, 48)),
    ((10, 64, 64, 64, 64, 784), torch.float32, "auto", ("resident", "resident"), (8, 4)),
])
def test_noalloc_steps_equal_the_plan_path(dims, dtype, wmode, paths, batches):
    for B, path in zip(batches, paths):
        report("noalloc", dims=len(dims) - 1, dtype=str(dtype), B=B, path=path)
        w0 = O.init_weights(dims, seed=B, init="xavier_uniform")
        x_in, _l, y = O.make_batch(dims, B, seed=B)
        m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=dtype, weight_update_mode=wmode,
                             hierarchical_policy_auto=False), device=DEV, weights=w0)
        m.initialize_batch(x_in.to(DEV), y.to(DEV))
        assert m.path == path
        xs, es, ws = [t.clone() for t in m.x], [t.clone() for t in m.e], [t.clone() for t in m.w]
        m.run_steps(T)
        nat.check(_noalloc(dims, B, xs, es, ws, nat.dtype_code(dtype), m.pred_split, nat.act_code("tanh"),
                           nat.WMODE[wmode], T))
        torch.cuda.synchronize()
        m.check_steps()
        for a, b in zip(m.x + m.e[:-1] + m.w, xs + es[:-1] + ws):
            assert torch.equal(a, b)


def test_noalloc_refuses_what_it_cannot_run():
    report("noalloc-refuse")
    # the wide net is not a whole-step net
    dims = (1000, 4096, 4096)
    P = [None] * 3
    rc = _noalloc(dims, 1024, P, P, P, nat.DT_BF16, 2, nat.act_code("tanh"), 0, 1)
    assert rc in (nat.ERR_NULL, nat.ERR_CONFIG)
    # a whole-step net whose f(x) buffers exceed the 8 MiB scratch (B = 4096)
    dims = (10, 64, 64, 784)
    t = [torch.zeros((d, 4096), device=DEV) for d in dims]
    ws = [torch.zeros((a, b), device=DEV) for a, b in zip(dims[:-1], dims[1:])]
    rc = _noalloc(dims, 4096, t, t, ws, nat.DT_F16, 3, nat.act_code("tanh"), 0, 1)
    assert rc == nat.ERR_SHAPE and "scratch" in nat.last_error()


@pytest.mark.parametrize("dims,dtype,B", [(D6, torch.float16, 128), ((10, 64, 64, 64, 784), torch.float32, 128)])
def test_noalloc_timeout_is_reported_until_checked(dims, dtype, B):
    """A spin limit of 0 (set from the host) makes every wait give up at its
    first unsatisfied poll; the kernels still run to their end.  The timeout
    word stays set across later calls until ipc_noalloc_check reports it, and
    calls at the default limit then check clean and match the plan path."""
    lib = nat.lib()
    report("noalloc-timeout", dims=len(dims) - 1, dtype=str(dtype), B=B)
    w0 = O.init_weights(dims, seed=5, init="xavier_uniform")
    x_in, _l, y = O.make_batch(dims, B, seed=5)
    m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=dtype, hierarchical_policy_auto=False), device=DEV,
               weights=w0)
    m.initialize_batch(x_in.to(DEV), y.to(DEV))
    x_init = [t.clone() for t in m.x]
    stream = nat.current_stream_handle(DEV)
    assert lib.ipc_noalloc_check(stream) in (nat.IPC_OK, nat.ERR_TIMEOUT)  # a clean start
    args = (nat.dtype_code(dtype), m.pred_split, nat.act_code("tanh"), nat.WMODE["gemm"])
    xs, es, ws = [t.clone() for t in m.x], [t.clone() for t in m.e], [t.clone() for t in m.w]
    try:
        lib.ipc_noalloc_set_spin_limit(0)
        nat.check(_noalloc(dims, B, xs, es, ws, *args, T))
        lib.ipc_noalloc_set_spin_limit(-1)
        nat.check(_noalloc(dims, B, xs, es, ws, *args, 1))  # a later call does not erase the report
        assert lib.ipc_noalloc_check(stream) == nat.ERR_TIMEOUT and "spin limit" in nat.last_error()
        assert lib.ipc_noalloc_check(stream) == nat.IPC_OK
    finally:
        lib.ipc_noalloc_set_spin_limit(-1)
    xs, es, ws = [t.clone() for t in x_init], [t.clone() for t in m.e], [w.to(DEV).clone() for w in w0]
    nat.check(_noalloc(dims, B, xs, es, ws, *args, T))
    assert lib.ipc_noalloc_check(stream) == nat.IPC_OK
    m.run_steps(T)
    m.check_steps()
    for a, b in zip(m.x + m.w, xs + ws):
        assert torch.equal(a, b)
