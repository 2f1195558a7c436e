"""Writes tests/golden/tiny_autograd.npz: torch CPU autograd (fp64) of the MoE
block on two tiny cases (up/down experts and reference single-linear experts).

torch is a third-party implementation independent of the oracle; routing
(top-k, ties to the lower index) is fixed from the fp64 logits, and the
load-balancing fraction cnt_e/(T*K) is a constant, as in the reference's
router_bwd_kernel (tmt-cuda/src/moe.cu:199-234). Run from the repo root:
    python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tiny_autograd.npz")


def case(seed, T, d, E, K, h, aux, zc):
    rng = np.random.default_rng(seed)
    hn = h if h > 0 else d
    arrs = {
        "X": rng.standard_normal((T, d)),
        "Wr": rng.standard_normal((E, d)) * 0.7,
        "Wu": rng.standard_normal((E, hn, d)) / np.sqrt(d),
        "dY": rng.standard_normal((T, d)),
        "bias": rng.standard_normal(E) * 0.3,
    }
    if h > 0:
        arrs["Wd"] = rng.standard_normal((E, d, h)) / np.sqrt(h)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=k not in ("dY", "bias"))
         for k, v in arrs.items()}
    logits = t["X"] @ t["Wr"].T + t["bias"]
    idx = np.argsort(-logits.detach().numpy(), axis=1, kind="stable")[:, :K]
    probs = torch.softmax(logits, dim=1)
    lse = torch.logsumexp(logits, dim=1)
    it = torch.tensor(idx)
    psel = probs.gather(1, it)
    gate = psel / psel.sum(1, keepdim=True)
    cnt = np.bincount(idx.ravel(), minlength=E)
    frac = torch.tensor(cnt / (T * K), dtype=torch.float64)
    aux_l = E * (probs.mean(0) * frac).sum()
    z_l = (lse ** 2).mean()
    Y = torch.zeros(T, d, dtype=torch.float64)
    for r in range(T):
        for j in range(K):
            e = int(idx[r, j])
            u = t["Wu"][e] @ t["X"][r]
            a = u * torch.sigmoid(u)
            o = t["Wd"][e] @ a if h > 0 else a
            Y[r] = Y[r] + gate[r, j] * o
    loss = (t["dY"] * Y).sum() + aux * aux_l + zc * z_l
    loss.backward()
    out = {k: v for k, v in arrs.items()}
    out.update(K=K, h=h, aux=aux, z=zc, loss=loss.item(), dX=t["X"].grad.numpy(),
               dWr=t["Wr"].grad.numpy(), dW_up=t["Wu"].grad.numpy())
    if h > 0:
        out["dW_down"] = t["Wd"].grad.numpy()
    return out


def main():
    res = {}
    for tag, args in (("h", (21, 9, 8, 5, 2, 6, 0.7, 0.3)), ("h0", (22, 7, 8, 4, 3, 0, 0.1, 1e-3))):
        for k, v in case(*args).items():
            res[f"{tag}_{k}"] = np.asarray(v)
    np.savez(OUT, **res)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
