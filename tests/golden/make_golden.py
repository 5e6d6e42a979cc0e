"""Writes the golden fixture of benchmark config 1 (tiny cache-latent DMLA forward, fp32).

Config 1: B=1, H=4, S=128, causal; Q [1,4,128,64] and a shared K_lat [1,128,64], all N(0,1)
from torch.Generator().manual_seed(0); V_lat = K_lat[..., :32]; softmax scale 1/sqrt(64).

The expected outputs are computed here in float64 by a brute-force row loop that follows the
exact three-pass softmax of the reference's vanilla kernel (csrc/attention/vanallia_attn.cu:33-82:
row max, row sum of exp, exp-weighted sum of V), independently of oracle/dmla_ref.py.  The
gradients dQ, dK_lat of sum(O * dO) come from torch.autograd in float64 on the same inputs.

Run:  python tests/golden/make_golden.py   (rewrites tests/golden/cfg1_tiny.npz)
"""
import os

import numpy as np
import torch

B, H, S, D, DV = 1, 4, 128, 64, 32
SCALE = 1.0 / 8.0


def brute_force(q, k):
    """q [B,H,S,D], k [B,S,D] float64 numpy -> o [B,H,S,DV], m, l [B,H,S]."""
    o = np.zeros((B, H, S, DV))
    m = np.zeros((B, H, S))
    l = np.zeros((B, H, S))
    for b in range(B):
        for h in range(H):
            for i in range(S):
                scores = np.array([SCALE * float(np.dot(q[b, h, i], k[b, j])) for j in range(i + 1)])
                row_max = scores.max()
                weights = np.exp(scores - row_max)
                row_sum = weights.sum()
                acc = np.zeros(DV)
                for j in range(i + 1):
                    acc += weights[j] * k[b, j, :DV]
                o[b, h, i] = acc / row_sum
                m[b, h, i] = row_max
                l[b, h, i] = row_sum
    return o, m, l


def main():
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, S, D, generator=gen, dtype=torch.float32)
    k_lat = torch.randn(B, S, D, generator=gen, dtype=torch.float32)
    do = torch.randn(B, H, S, DV, generator=gen, dtype=torch.float32)
    o, m, l = brute_force(q.double().numpy(), k_lat.double().numpy())

    qx = q.double().requires_grad_(True)
    kx = k_lat.double().requires_grad_(True)
    s = SCALE * torch.matmul(qx, kx.unsqueeze(1).transpose(-1, -2))
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    out = torch.matmul(torch.softmax(s, dim=-1), kx[..., :DV].unsqueeze(1))
    (out * do.double()).sum().backward()

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg1_tiny.npz")
    np.savez_compressed(
        path,
        q=q.numpy(), k_lat=k_lat.numpy(), do=do.numpy(),
        o=o.astype(np.float32), m=m.astype(np.float32), l=l.astype(np.float32),
        lse=(m + np.log(l)).astype(np.float32),
        dq=qx.grad.numpy().astype(np.float32), dk_lat=kx.grad.numpy().astype(np.float32),
        scale=np.float64(SCALE), d_v=np.int64(DV),
    )
    print("wrote", path, "max |o_autograd - o_loop| =", float((out.detach().numpy() - o).__abs__().max()))


if __name__ == "__main__":
    main()
