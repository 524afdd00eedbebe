"""Write golden trajectories of the reference optimizer (run in the build container only).

What no closed form pins -- the free-running multi-step trajectories of
IFKFAC.step on the demo / canary models -- is recorded here by running the
reference package itself (Gsend/ifkfac, mounted at /root/reference) on the
CPU.  The output is data only: per-step losses and final parameters, saved as
``reference_trajectories.npz`` next to this script.  The reference never
travels with the repository; this script is not run by the tests.

Configurations (seeded exactly as below):
  demo_fp32 / demo_bf16: Linear(128,256)-ReLU-Linear(256,10), batch 256,
      x ~ N(0,1), labels uniform over 10 classes (generator seed 0, model seed 0),
      cross-entropy, IFKFAC(lr=1e-3, damping=1e-2, factor_update_freq=1,
      momentum=0.9, use_true_bf16=False/True), 100 steps.
  canary: the 16-32-32-8 ReLU MLP of the reference's test_basic.py (seed 42),
      MSE, lr=1e-2, damping=1e-2, freq=10, 60 steps (initial forward included).
  canary_bias: 8-16-4 ReLU MLP with bias (seed 0), MSE, lr=1e-2, freq=5, 40 steps.
"""
import contextlib
import io
import os
import sys

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"


def demo(IFKFAC, use_bf16, steps=100, device="cpu"):
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(128, 256), nn.ReLU(), nn.Linear(256, 10))
    g = torch.Generator().manual_seed(0)
    x = torch.randn(256, 128, generator=g)
    y = torch.randint(0, 10, (256,), generator=g)
    init = [p.detach().clone().numpy() for p in model.parameters()]
    model, x, y = model.to(device), x.to(device), y.to(device)
    opt = IFKFAC(model, lr=1e-3, damping=1e-2, factor_update_freq=1, momentum=0.9,
                 use_true_bf16=use_bf16)
    losses = []
    for _ in range(steps):
        opt.zero_grad()
        loss = F.cross_entropy(model(x), y)
        loss.backward()
        opt.step()
        losses.append(loss.item())
    return (np.array(losses), [p.detach().cpu().numpy() for p in model.parameters()], init,
            x.cpu().numpy(), y.cpu().numpy())


def canary(IFKFAC, device="cpu"):
    torch.manual_seed(42)
    model = nn.Sequential(nn.Linear(16, 32), nn.ReLU(), nn.Linear(32, 32), nn.ReLU(),
                          nn.Linear(32, 8))
    g = torch.Generator().manual_seed(0)
    X = torch.randn(128, 16, generator=g)
    Y = torch.randn(128, 8, generator=g)
    model, X, Y = model.to(device), X.to(device), Y.to(device)
    opt = IFKFAC(model, lr=1e-2, damping=1e-2, factor_update_freq=10)
    losses = [F.mse_loss(model(X), Y).item()]
    for _ in range(60):
        loss = F.mse_loss(model(X), Y)
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    losses.append(F.mse_loss(model(X), Y).item())
    return np.array(losses)


def canary_bias(IFKFAC, device="cpu"):
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(8, 16, bias=True), nn.ReLU(), nn.Linear(16, 4, bias=True))
    g = torch.Generator().manual_seed(1)
    X = torch.randn(64, 8, generator=g)
    Y = torch.randn(64, 4, generator=g)
    model, X, Y = model.to(device), X.to(device), Y.to(device)
    opt = IFKFAC(model, lr=1e-2, damping=1e-2, factor_update_freq=5)
    losses = [F.mse_loss(model(X), Y).item()]
    for _ in range(40):
        loss = F.mse_loss(model(X), Y)
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    losses.append(F.mse_loss(model(X), Y).item())
    return np.array(losses)


def main():
    sys.path.insert(0, REF)
    from ifkfac import IFKFAC  # the reference package
    torch.set_num_threads(1)
    out = {}
    with contextlib.redirect_stdout(io.StringIO()):
        for tag, bf in (("demo_fp32", False), ("demo_bf16", True)):
            losses, final, init, x, y = demo(IFKFAC, bf)
            out[f"{tag}_losses"] = losses
            for i, w in enumerate(final):
                out[f"{tag}_final_{i}"] = w
        out["canary_losses"] = canary(IFKFAC)
        out["canary_bias_losses"] = canary_bias(IFKFAC)
    out["torch_version"] = np.array(torch.__version__)
    path = os.path.join(HERE, "reference_trajectories.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)
    for k in ("demo_fp32_losses", "demo_bf16_losses", "canary_losses", "canary_bias_losses"):
        v = out[k]
        print(k, v[:3], "...", v[-3:])


if __name__ == "__main__":
    main()
