"""KDA chunk oracle in torch on the CPU (test and CPU-baseline infrastructure only).

``chunk_kda`` restates ``naive_chunk_kda`` (``/root/reference/ops_kda.py:340-536``)
with torch tensor operations on the CPU, the same steps as ``oracle.kda.chunk_kda``
(right-pad to the chunk, ``:375-382``; in-chunk cumsum of the clamped gate,
``:388-394``; the per-column build of A with ``clamp(max=50)``, ``:409-417``; the
unit-lower triangular solve and ``(A + I) diag(beta)``, ``:418-421``; ``w``/``u``,
``:423-424``; the sequential chunk loop, ``:509-535``). It exists so that the
CPU baseline runs on torch's intra-op thread pool (``torch.set_num_threads``),
as the reference's own CPU path does; ``tests/test_oracle_kda.py`` holds it to
``oracle.kda.chunk_kda``.
"""

from __future__ import annotations

import torch


def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, chunk_size=64,
              g_clamp_min=-10.0, dtype=torch.float32):
    """Chunkwise WY form on CPU tensors (or arrays); returns ``(o [B,T,HV,V],
    S [B,HV,K,V])`` in ``dtype``."""
    t = lambda x: torch.as_tensor(x).to(dtype)  # noqa: E731
    q, k, v, g, beta = (t(x) for x in (q, k, v, g, beta))
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    G = HV // H
    if scale is None:
        scale = K ** -0.5
    q = q.repeat_interleave(G, dim=2) * scale
    k = k.repeat_interleave(G, dim=2)
    S = torch.zeros(B, HV, K, V, dtype=dtype)
    if initial_state is not None:
        S = S + t(initial_state)
    if T == 0:
        return torch.zeros(B, 0, HV, V, dtype=dtype), S
    C = chunk_size
    pad = (-T) % C
    if pad:
        q, k, v, g = (torch.nn.functional.pad(x, (0, 0, 0, 0, 0, pad)) for x in (q, k, v, g))
        beta = torch.nn.functional.pad(beta, (0, 0, 0, pad))
    NT = (T + pad) // C

    def chunks(x):  # [B, Tp, HV, ...] -> [B, HV, NT, C, ...]
        return x.reshape(B, NT, C, HV, *x.shape[3:]).movedim(3, 1)

    q, k, v, g = (chunks(x) for x in (q, k, v, g))
    beta = chunks(beta)
    if g_clamp_min > float('-inf'):
        g = g.clamp(min=g_clamp_min)
    g = g.cumsum(dim=-2)
    cap = torch.tensor(50.0, dtype=dtype)
    A = torch.zeros(B, HV, NT, C, C, dtype=dtype)
    for i in range(C - 1):
        gd = torch.minimum(g[..., i + 1:, :] - g[..., i:i + 1, :], cap)
        A[..., i + 1:, i] = (k[..., i + 1:, :] * gd.exp() * k[..., i:i + 1, :]).sum(-1)
    A = -(A * beta[..., None])
    eye = torch.eye(C, dtype=dtype)
    X = torch.linalg.solve_triangular(eye - A, A, upper=False, unitriangular=True)
    A = (X + eye) * beta[..., None, :]
    w = A @ (g.exp() * k)
    u = A @ v
    Aqk = torch.zeros(B, HV, NT, C, C, dtype=dtype)
    for c in range(C):
        diff = torch.minimum(g[..., c:, :] - g[..., c:c + 1, :], cap)
        Aqk[..., c:, c] = (q[..., c:, :] * diff.exp() * k[..., c:c + 1, :]).sum(-1)
    o = torch.zeros(B, HV, NT, C, V, dtype=dtype)
    for n in range(NT):
        qn, kn, un, gn, wn = q[:, :, n], k[:, :, n], u[:, :, n], g[:, :, n], w[:, :, n]
        vn = un - wn @ S
        o[:, :, n] = (qn * gn.exp()) @ S + Aqk[:, :, n] @ vn
        glast = gn[:, :, -1]
        S = S * glast.exp()[..., None]
        S = S + ((glast[:, :, None, :] - gn).exp() * kn).transpose(-1, -2) @ vn
    o = o.reshape(B, HV, NT * C, V).transpose(1, 2)[:, :T]
    return o.contiguous(), S
