"""SVD low-rank SwiGLU FFN oracle (numpy, float64).  Test infrastructure only.

Factors follow SVDFactorSparseFFN.refresh_svd (rte/layers.py:437-444): for an input-major
weight W (d x F), A = U[:, :r] S[:r] and B = Vh[:r]; up_hat = (x A_up) B_up
(rte/layers.py:593-596).  BASELINE configs[3] uses the rank-r factors as the weights of
all three projections (down: W_down^T = U_dn S_dn V_dn^T)."""

from __future__ import annotations

import numpy as np

from oracle.swiglu import sigmoid, silu


def svd_ffn_fwd(x, us_up, us_gate, v_up, v_gate, v_dn, us_dn):
    x = np.asarray(x, np.float64)
    a_up = x @ us_up
    a_gate = x @ us_gate
    up = a_up @ v_up.T
    gate = a_gate @ v_gate.T
    z = up * silu(gate)
    b = z @ v_dn
    y = b @ us_dn.T
    return y, dict(a_up=a_up, a_gate=a_gate, up=up, gate=gate, z=z, b=b)


def svd_ffn_bwd(dy, x, us_up, us_gate, v_up, v_gate, v_dn, us_dn, c):
    dy = np.asarray(dy, np.float64)
    x = np.asarray(x, np.float64)
    db = dy @ us_dn
    dus_dn = dy.T @ c["b"]
    dz = db @ v_dn.T
    dv_dn = c["z"].T @ db
    s = sigmoid(c["gate"])
    dup = dz * c["gate"] * s
    dgate = dz * c["up"] * s * (1.0 + c["gate"] * (1.0 - s))
    da_up = dup @ v_up
    da_gate = dgate @ v_gate
    dv_up = dup.T @ c["a_up"]
    dv_gate = dgate.T @ c["a_gate"]
    dx = da_up @ us_up.T + da_gate @ us_gate.T
    return dict(dx=dx, dus_up=x.T @ da_up, dus_gate=x.T @ da_gate, dv_up=dv_up, dv_gate=dv_gate, dv_dn=dv_dn,
                dus_dn=dus_dn)
