"""fp32 torch reference of the MoE block for the full-size GPU parity tests.

Used where the CPU oracle would take minutes (c2/c3 backward): the same maths
in fp32 with torch autograd, given the routing (idx) that the router parity
test has already matched bit for bit against the oracle. Gates stay
differentiable (softmax -> gather -> renormalise); the load-balancing
fraction cnt/(T*K) is a constant, as in the reference's router_bwd_kernel
(tmt-cuda/src/moe.cu:199-234). Only fp32 2-D matmuls are used.
"""
import torch


def moe_reference(X, Wr, W_up, W_down, idx, dY, h, bias=None, Y_in=None, beta=0.0,
                  aux_coef=0.0, z_coef=0.0, need_grads=True):
    """All tensors fp32 on one device; idx int64 [T, K]. Returns dict with Y
    and, when need_grads, dX, dWr, dW_up, dW_down (None where absent)."""
    T, d = X.shape
    E, K = W_up.shape[0], idx.shape[1]
    X = X.detach().clone().requires_grad_(need_grads)
    Wr = None if Wr is None else Wr.detach().clone().requires_grad_(need_grads)
    W_up = W_up.detach().clone().requires_grad_(need_grads)
    W_down = None if W_down is None else W_down.detach().clone().requires_grad_(need_grads)
    if E > 1:
        logits = X @ Wr.t()
        if bias is not None:
            logits = logits + bias
        probs = torch.softmax(logits, dim=1)
        lse = torch.logsumexp(logits, dim=1)
        psel = probs.gather(1, idx)
        gate = psel / psel.sum(1, keepdim=True)
        cnt = torch.bincount(idx.reshape(-1), minlength=E).to(X.dtype)
        frac = cnt / (T * K)
        aux = E * (probs.mean(0) * frac).sum()
        z = (lse * lse).mean()
    else:
        gate = torch.ones(T, 1, dtype=X.dtype, device=X.device)
        aux = z = torch.zeros((), dtype=X.dtype, device=X.device)
    Y = torch.zeros(T, d, dtype=X.dtype, device=X.device)
    if Y_in is not None and beta != 0.0:
        Y = Y + beta * Y_in
    for e in range(E):
        rows, js = torch.nonzero(idx == e, as_tuple=True)
        if rows.numel() == 0:
            continue
        xe = X[rows]
        u = xe @ W_up[e].t()
        a = u * torch.sigmoid(u)
        o = a @ W_down[e].t() if h > 0 else a
        Y = Y.index_add(0, rows, gate[rows, js].unsqueeze(1) * o)
    out = {"Y": Y.detach(), "aux": float(aux.detach()), "z": float(z.detach())}
    if need_grads:
        loss = (dY * Y).sum() + aux_coef * aux + z_coef * z
        loss.backward()
        out["dX"] = X.grad
        out["dWr"] = None if Wr is None else Wr.grad
        out["dW_up"] = W_up.grad
        out["dW_down"] = None if W_down is None else W_down.grad
    return out
