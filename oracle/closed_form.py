"""Independent float64 closed forms that pin the oracle (test infrastructure).

These do not reuse the oracle's formulas; they restate the mathematics the reference's
own CPU tests use as ground truth:

* attention weights are the softmax of the compressed logits ``n asinh(s/c)`` with a sink
  column (tests/test_components.py:27-40; paper/paper.tex:408-440), so the forward is a
  textbook softmax attention and its gradient comes from torch float64 autograd;
* the head's gradient is the gradient of the true NLL ``-mean log softmax(n asinh(z/c))_t``
  (tests/test_components.py:43-56; src/algebraic/evaluation.py:13-23), again by autograd.
"""

import math

import numpy as np


def _torch():
    import torch
    return torch


def attention_closed_form(q, k, v, sink_logit, do, *, n=16, c=8.0):
    """(o, dq, dk, dv, dsink) from torch float64 autograd of softmax(n*asinh(s/c)) attention."""
    torch = _torch()
    B, H, T, D = q.shape
    tq, tk, tv = (torch.tensor(np.asarray(a, np.float64), requires_grad=True) for a in (q, k, v))
    ts = None
    if sink_logit is not None:
        ts = torch.tensor(np.asarray(sink_logit, np.float64), requires_grad=True)
    s = torch.einsum("bhqd,bhkd->bhqk", tq, tk) / math.sqrt(D)
    logits = n * torch.asinh(s / c)
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    logits = logits.masked_fill(~mask, float("-inf"))
    if ts is not None:
        sb = ts.reshape(-1).expand(H) if ts.numel() in (1, H) else None
        col = (n * torch.asinh(sb / c)).reshape(1, H, 1, 1).expand(B, H, T, 1)
        full = torch.cat([logits, col], dim=-1)
        p = torch.softmax(full, dim=-1)[..., :T]
    else:
        p = torch.softmax(logits, dim=-1)
    o = torch.einsum("bhqk,bhkd->bhqd", p, tv)
    loss = (o * torch.tensor(np.asarray(do, np.float64))).sum()
    loss.backward()
    return (o.detach().numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy(),
            None if ts is None else ts.grad.numpy())


def head_closed_form(h, E, targets, g=1.0, *, n=8, c=2.0):
    """(nll_mean, pt, dh, dE) from torch float64 autograd of the true NLL."""
    torch = _torch()
    th = torch.tensor(np.asarray(h, np.float64), requires_grad=True)
    tE = torch.tensor(np.asarray(E, np.float64), requires_grad=True)
    z = th @ tE.T
    a = n * torch.asinh(z / c)
    logp = torch.log_softmax(a, dim=-1)
    t = torch.tensor(np.asarray(targets, np.int64))
    lpt = logp.gather(1, t[:, None])[:, 0]
    nll = -lpt.mean()
    (nll * g).backward()
    return nll.item(), lpt.exp().detach().numpy(), th.grad.numpy(), tE.grad.numpy()


def attention_brute_force(q, k, v, sink_logit, *, n=16, c=8.0):
    """Pure-Python loops over (b, h, i, j) for tiny shapes: o_i = sum_j P_ij v_j."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, H, T, D = q.shape
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            for i in range(T):
                logits = []
                for j in range(i + 1):
                    s = sum(q[b, h, i, d] * k[b, h, j, d] for d in range(D)) / math.sqrt(D)
                    logits.append(n * math.asinh(s / c))
                mx = max(logits)
                if sink_logit is not None:
                    sb = np.asarray(sink_logit, np.float64).reshape(-1)
                    sb = sb[h] if sb.size == H else sb[0]
                    lb = n * math.asinh(sb / c)
                    mx = max(mx, lb)
                    denom = math.exp(lb - mx)
                else:
                    denom = 0.0
                ws = [math.exp(a - mx) for a in logits]
                denom += sum(ws)
                for j in range(i + 1):
                    for d in range(D):
                        out[b, h, i, d] += ws[j] / denom * v[b, h, j, d]
    return out
