"""rdv_mlp_train_step_static (the training step with its workspace in a
static device array, for callers that cannot allocate) against
rdv_mlp_train_step (caller workspace), both called through the C ABI.

The two entry points run the same kernels on the same inputs and reduce dW in
the same fixed order, so loss and every gradient must agree bit for bit.  Two
calls in a row, the second on fewer points, check that nothing the first call
left in the shared scratch leaks into the second."""
import ctypes as C

import pytest
import torch

import rdv_project_amd as rdv
from rdv_project_amd import _chain, _lib
from rdv_project_amd import workloads as WL

pytestmark = pytest.mark.gpu


def _chain_of(layers):
    m = None
    for i, (w, b) in enumerate(layers):
        lin = rdv.linear(w.cuda(), b.cuda(), f16=True)
        m = lin if m is None else m >> lin
        if i + 1 < len(layers):
            m = m >> rdv.relu
    return m


def _grads(p):
    return [(torch.full((l.OUT, l.IN), float("nan"), device="cuda"), torch.full((l.OUT,), float("nan"), device="cuda"))
            for l in p.layers]


def _run(lib, p, packed, x, t, static):
    n = int(x.shape[0])
    loss = torch.full((), float("nan"), device="cuda")
    grads = _grads(p)
    dws = _lib.void_ptr_array([g[0].data_ptr() for g in grads])
    dbs = _lib.void_ptr_array([g[1].data_ptr() for g in grads])
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if static:
        rc = lib.rdv_mlp_train_step_static(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.c_void_p(x.data_ptr()),
                                           C.c_void_p(t.data_ptr()), C.c_int64(n), C.c_void_p(loss.data_ptr()),
                                           dws, dbs, stream)
    else:
        nbytes = lib.rdv_mlp_train_workspace_bytes(C.byref(p.desc), C.c_int64(n))
        assert nbytes > 0, _lib.last_error()
        ws = torch.empty(int(nbytes) + 256, dtype=torch.uint8, device="cuda")
        off = (-ws.data_ptr()) % 256
        rc = lib.rdv_mlp_train_step(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.c_void_p(x.data_ptr()),
                                    C.c_void_p(t.data_ptr()), C.c_int64(n), C.c_void_p(ws.data_ptr() + off),
                                    C.c_int64(nbytes), C.c_void_p(loss.data_ptr()), dws, dbs, stream)
    _lib.check(rc, "train step")
    torch.cuda.synchronize()
    return loss.cpu(), [(dw.cpu(), db.cpu()) for dw, db in grads]


def _setup(n):
    x, t, layers = WL.c5(n)
    layers = [(w, torch.randn(w.shape[0], generator=torch.Generator().manual_seed(40 + i)) * 0.1)
              for i, (w, _) in enumerate(layers)]
    m = _chain_of(layers)
    p = _chain.plan_chain(m, 32)
    return p, _chain.packed_params(m, p), x.cuda().contiguous(), t.cuda().contiguous()


def test_static_scratch_matches_caller_workspace():
    lib = _lib.load()
    p, packed, x, t = _setup(2000)
    for n in (2000, 777):  # the second call is smaller: stale scratch from the first must not matter
        xs, ts = x[:n].contiguous(), t[:n].contiguous()
        ref_loss, ref_grads = _run(lib, p, packed, xs, ts, static=False)
        loss, grads = _run(lib, p, packed, xs, ts, static=True)
        assert torch.isfinite(loss) and torch.equal(loss, ref_loss), f"n={n}: loss {loss} vs {ref_loss}"
        for l, ((dw, db), (rw, rb)) in enumerate(zip(grads, ref_grads)):
            assert torch.isfinite(dw).all() and torch.isfinite(db).all(), f"n={n}: layer {l} not written"
            assert torch.equal(dw, rw) and torch.equal(db, rb), f"n={n}: layer {l} differs"


def test_static_scratch_rejects_oversize_workspace():
    lib = _lib.load()
    n = 1 << 20  # needs far more workspace than the static scratch holds; rejected before any launch
    p, packed, x, t = _setup(n)  # full-size buffers all the same, so no pointer is ever short
    need = lib.rdv_mlp_train_workspace_bytes(C.byref(p.desc), C.c_int64(n))
    assert need > _lib.TRAIN_STATIC_SCRATCH_BYTES
    loss = torch.empty((), device="cuda")
    grads = _grads(p)
    dws = _lib.void_ptr_array([g[0].data_ptr() for g in grads])
    dbs = _lib.void_ptr_array([g[1].data_ptr() for g in grads])
    rc = lib.rdv_mlp_train_step_static(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.c_void_p(x.data_ptr()),
                                       C.c_void_p(t.data_ptr()), C.c_int64(n), C.c_void_p(loss.data_ptr()), dws, dbs,
                                       C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == _lib.RDV_ERR_WORKSPACE
    assert "static scratch" in _lib.last_error()
