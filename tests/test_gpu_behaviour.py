"""Training-behaviour tests of the reference, run on the GPU through the drop-in LuminaV.

* End-to-end MLP training (optimizer/tests/test_end_to_end_training.py:12-79): the loss falls
  over 10 steps and every parameter moves, for every buffer mode, in fp32 and bf16, unfused and
  bucket-fused.
* bf16 stochastic-rounding post-spike decay (test_end_to_end_training.py:477-534,
  core_tests.rs:239-326): after one gradient spike of 100 and 599 zero gradients, the bf16
  exp_avg_sq mean stays above 8 with round-to-nearest (it freezes) and falls below 6.5 with
  stochastic rounding, for buffer 2 and T2 with master weights none and semi. With
  master_weights="full" the state is fp32.
* Fused lagged-scale EMA vs two-pass statistics (eval/modules/parity_audit.py:9-107): on the ill-
  conditioned quadratic 0.5 (w0^2 + 1000 w1^2) from w = (10, 1) with the radial bound, both
  pass shapes converge below 1e-4 and the fused one needs at most a few percent more steps.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


class SimpleMLP(nn.Module):
    def __init__(self, in_features: int = 64, hidden: int = 128, out_features: int = 10):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(in_features, hidden), nn.ReLU(), nn.Linear(hidden, hidden), nn.ReLU(),
                                 nn.Linear(hidden, out_features))

    def forward(self, x):
        return self.net(x)


@pytest.mark.parametrize("fuse", [False, True], ids=["unfused", "fused"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("buffer", [2, 1, "T2", "T1"])
def test_mlp_loss_decreases(buffer, dtype, fuse):
    _need_gpu()
    from luminamoon_amd import LuminaV

    torch.manual_seed(42)
    model = SimpleMLP().cuda().to(dtype)
    opt = LuminaV(model.parameters(), lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01, buffer=buffer, bound=True,
                  cautious=True, fuse_tensors=fuse)
    x = torch.randn(32, 64, device="cuda", dtype=dtype)
    target = torch.randn(32, 10, device="cuda", dtype=dtype)
    initial = [p.detach().clone() for p in model.parameters()]
    losses = []
    for _ in range(10):
        opt.zero_grad()
        loss = nn.functional.mse_loss(model(x).float(), target.float())
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0], f"loss did not decrease: {losses}"
    for i, (p0, p) in enumerate(zip(initial, model.parameters())):
        assert (p.detach().float() - p0.float()).abs().max().item() > 0.0, f"parameter {i} was not updated"


@pytest.mark.parametrize("master", ["none", "semi"])
@pytest.mark.parametrize("buffer", [2, "T2"])
def test_bf16_sr_vs_rne_post_spike_decay(buffer, master):
    _need_gpu()
    from luminamoon_amd import LuminaV

    p_rne = nn.Parameter(torch.ones(256, dtype=torch.bfloat16, device="cuda"))
    p_sr = nn.Parameter(torch.ones(256, dtype=torch.bfloat16, device="cuda"))
    # state_precision="param": bf16 exp_avg_sq, the reference's default for bf16 params
    opt_rne = LuminaV([p_rne], lr=1e-3, buffer=buffer, master_weights=master, stochastic_rounding=False,
                      state_precision="param")
    opt_sr = LuminaV([p_sr], lr=1e-3, buffer=buffer, master_weights=master, stochastic_rounding=True,
                     state_precision="param")
    spike = torch.full_like(p_rne, 100.0)
    zeros = torch.zeros_like(p_rne)
    for i in range(600):
        g = spike if i == 0 else zeros
        p_rne.grad = g.clone()
        p_sr.grad = g.clone()
        opt_rne.step()
        opt_sr.step()
    v_rne = opt_rne.state[p_rne]["exp_avg_sq"]
    v_sr = opt_sr.state[p_sr]["exp_avg_sq"]
    assert v_rne.dtype == torch.bfloat16 and v_sr.dtype == torch.bfloat16
    v_rne, v_sr = v_rne.float(), v_sr.float()
    assert torch.isfinite(v_sr).all() and bool((v_sr >= 0.0).all())
    assert float(v_rne.mean()) > 8.0, f"RNE exp_avg_sq should freeze above 8, got {float(v_rne.mean())}"
    assert float(v_sr.mean()) < 6.5, f"SR exp_avg_sq should decay below 6.5, got {float(v_sr.mean())}"


def test_master_full_keeps_fp32_state():
    _need_gpu()
    from luminamoon_amd import LuminaV

    p = nn.Parameter(torch.ones(64, dtype=torch.bfloat16, device="cuda"))
    opt = LuminaV([p], lr=1e-3, buffer=2, master_weights="full", stochastic_rounding=True, state_precision="param")
    p.grad = torch.ones_like(p)
    opt.step()
    assert opt.state[p]["exp_avg_sq"].dtype == torch.float32


def _quadratic_steps(buffer, fused: bool, max_steps: int = 1000, tol: float = 1e-4):
    from luminamoon_amd import LuminaV

    w = nn.Parameter(torch.tensor([10.0, 1.0], device="cuda"))
    opt = LuminaV([w], lr=0.02, buffer=buffer, bound_type="radial", cautious=True, weight_decay=0.0,
                  fused_single_pass=fused)
    scale = torch.tensor([1.0, 1000.0], device="cuda")
    loss = None
    for t in range(1, max_steps + 1):
        w.grad = (scale * w.detach()).clone()
        opt.step()
        loss = float(0.5 * (w.detach() ** 2 * scale).sum())
        if loss < tol:
            return t, loss
    return max_steps, loss


@pytest.mark.parametrize("buffer", [1, 2])
def test_fused_ema_vs_two_pass_on_quadratic(buffer):
    _need_gpu()
    steps_two, loss_two = _quadratic_steps(buffer, fused=False)
    steps_fused, loss_fused = _quadratic_steps(buffer, fused=True)
    print(f"[quadratic] buffer={buffer}: two-pass {steps_two} steps (loss {loss_two:.2e}), "
          f"fused EMA {steps_fused} steps (loss {loss_fused:.2e})", flush=True)
    assert loss_two < 1e-4 and loss_fused < 1e-4, "both pass shapes must converge"
    assert steps_fused <= steps_two * 1.05 + 2, f"fused EMA needs {steps_fused} steps vs two-pass {steps_two}"
