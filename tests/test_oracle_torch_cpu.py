"""The torch-CPU restatement that bench.py times as its CPU baseline
(oracle/torch_cpu.py) against the numpy oracle it restates: same seeded
inputs, the stated tolerances.  CPU only."""
import numpy as np
import torch

from oracle import mlp as O
from oracle import render as R
from oracle import torch_cpu as TC
from oracle import train as T
from oracle import winograd as W
from rdv_project_amd import workloads as WL


def test_mlp_forward_c2_shape():
    x, layers = WL.c2(4096)
    acts = ["relu"] * 3 + ["none"]
    y = TC.mlp_forward(x, TC.pack_layers(layers), acts, encoding=(WL.C2_OCTAVES, WL.C2_PAD)).numpy()
    ref = O.mlp_forward(x.numpy(), [(w.numpy(), b.numpy()) for w, b in layers], acts, ["f16"] * 4,
                        encoding=(WL.C2_OCTAVES, WL.C2_PAD))
    assert O.within_tolerance(y, ref).all()


def test_mlp_forward_c1_shape_with_bias():
    x, layers = WL.c1(2048)
    layers = [(w, torch.linspace(-0.2, 0.3, w.shape[0])) for w, _ in layers]
    acts = ["relu"] * 4 + ["none"]
    y = TC.mlp_forward(x, TC.pack_layers(layers), acts).numpy()
    ref = O.mlp_forward(x.numpy(), [(w.numpy(), b.numpy()) for w, b in layers], acts, ["f16"] * 5)
    assert O.within_tolerance(y, ref).all()


def test_conv3x3_matches_direct_conv():
    x, w, _ = WL.c3(16, 12, 16, 32)
    y = TC.conv3x3(x.float(), w.float(), relu=True).numpy()[0].transpose(1, 2, 0)
    ref = W.direct_conv(x.float().numpy()[0].transpose(1, 2, 0), w.float().numpy().transpose(2, 3, 1, 0), relu=True)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_render_ea_matches_oracle():
    layers = WL.c4_mlp()
    rays = R.camera_rays(24, 16, WL.c4_pose().numpy()).reshape(-1, 6)
    img = TC.render_ea(torch.from_numpy(rays.astype(np.float32)), TC.pack_layers(layers), 64).numpy()
    ref = R.render_ea(rays, [(w.numpy(), b.numpy()) for w, b in layers], 64)
    assert (ref > 0).any()
    np.testing.assert_allclose(img, ref, rtol=1e-3, atol=1e-5)


def test_train_step_matches_oracle():
    x, t, layers = WL.c5(512)
    params = [(w.clone().requires_grad_(True), torch.full((w.shape[0],), 0.05).requires_grad_(True))
              for w, _ in layers]
    loss = TC.train_step(x.float(), t, params)
    ref_loss, ref_grads = T.mse_grads(x.float().numpy(), [(w.detach().numpy(), b.detach().numpy())
                                                          for w, b in params], t.numpy())
    assert abs(loss.item() - ref_loss) <= 1e-4 * ref_loss
    for (w, b), (rw, rb) in zip(params, ref_grads):
        ew = np.linalg.norm(w.grad.numpy() - rw) / np.linalg.norm(rw)
        eb = np.linalg.norm(b.grad.numpy() - rb) / np.linalg.norm(rb)
        assert ew <= 1e-2 and eb <= 1e-2, (ew, eb)
