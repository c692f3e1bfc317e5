"""gn_dense_backward_noalloc (static device scratch, no allocation) against
gn_dense_backward (caller workspace + context scratch): identical results on
two calls in a row, the second with a smaller input, and the size limit."""
import ctypes as C

import numpy as np
import pytest

from gpuutil import DBuf, log

pytestmark = pytest.mark.gpu


def _case(lib, check, dev, B, I, O, act, ptr, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(B, I)).astype(np.float32)
    W = (rng.normal(size=(O, I)) * 0.05).astype(np.float32)
    out = rng.uniform(0.01, 0.99, size=(B, O)).astype(np.float32)
    if ptr:  # softmax rows for the Jacobian path
        out = out / out.sum(1, keepdims=True)
    g = rng.normal(size=(B, O)).astype(np.float32)
    dx, dW, do, dg = DBuf(dev, x), DBuf(dev, W), DBuf(dev, out), DBuf(dev, g)
    res = []
    for noalloc in (False, True):
        gW = DBuf(dev, np.zeros((O, I), np.float32))
        gB = DBuf(dev, np.zeros(O, np.float32))
        gin = DBuf(dev, np.zeros((B, I), np.float32))
        scale = C.c_float(np.float32(1.0) / np.float32(B))
        if noalloc:
            check(dev.h, lib.gn_dense_backward_noalloc(dev.h, dx.p, dW.p, do.p, dg.p, gW.p, gB.p, gin.p,
                                                       B, I, O, act, ptr, scale))
        else:
            dz = DBuf(dev, np.zeros((B, O), np.float32))
            check(dev.h, lib.gn_dense_backward(dev.h, dx.p, dW.p, do.p, dg.p, gW.p, gB.p, gin.p, dz.p,
                                               B, I, O, act, ptr, scale))
        res.append((gW.get(), gB.get(), gin.get()))
    for a, b, name in zip(res[0], res[1], ("gradW", "gradB", "gin")):
        np.testing.assert_array_equal(a, b, err_msg=name)
    log(f"  noalloc B={B} in={I} out={O} act={act}: identical to the workspace entry point")


@pytest.mark.parametrize("act,ptr", [(1, 0), (4, 1)])
def test_dense_backward_noalloc_matches_workspace_entry(gn, dev, act, ptr):
    from goneuron_amd._lib import lib, check
    # the second call is smaller: the array keeps the first call's contents
    _case(lib(), check, dev, 1024, 4096, 4096, act, ptr, 1)
    _case(lib(), check, dev, 37, 91, 53, act, ptr, 2)


def test_dense_backward_noalloc_rejects_oversize(gn, dev):
    from goneuron_amd._lib import lib, GNError, check
    p = C.c_void_p(16)  # never dereferenced: the size check runs first
    rc = lib().gn_dense_backward_noalloc(dev.h, p, p, p, p, p, p, p, 4097, 8, 1024, 1, 0,
                                         C.c_float(1.0))
    assert rc == -1
    assert b"exceeds the static scratch limit" in lib().gn_last_error(dev.h)
