"""Brute-force scalar restatements of the triangle ops for tiny shapes.

Plain Python loops over ``math``; no numpy arithmetic, no matmul, no
broadcasting. These exist to pin the vectorised oracle: a transposed
operand, a wrong contraction index or a dropped bias term in the oracle
shows up as a mismatch against these loops.
"""

from __future__ import annotations

import math


def ln_vec(x, w, b, eps=1e-5):
    n = len(x)
    mean = sum(x) / n
    var = sum((v - mean) ** 2 for v in x) / n
    inv = 1.0 / math.sqrt(var + eps)
    return [(x[c] - mean) * inv * w[c] + b[c] for c in range(n)]


def sig(v):
    return 1.0 / (1.0 + math.exp(-v)) if v >= 0 else math.exp(v) / (1.0 + math.exp(v))


def matvec_torch(w, x):
    """``W x`` for a torch-layout weight ``W[out][in]``."""
    return [sum(w[o][i] * x[i] for i in range(len(x))) for o in range(len(w))]


def trimul(z, mask, p, outgoing, eps=1e-5):
    """Algorithm 12/13 with torch-layout weights (``p`` holds nested lists)."""
    n = len(z)
    ln_in, ln_out = p["layer_norm_in"], p["layer_norm_out"]
    zn = [[ln_vec(z[i][j], ln_in["weight"], ln_in["bias"], eps) for j in range(n)] for i in range(n)]

    def proj(pn, gn, i, j):
        pv = matvec_torch(p[pn]["weight"], zn[i][j])
        gv = matvec_torch(p[gn]["weight"], zn[i][j])
        return [mask[i][j] * sig(gv[c]) * pv[c] for c in range(len(pv))]

    a = [[proj("linear_a_p", "linear_a_g", i, j) for j in range(n)] for i in range(n)]
    b = [[proj("linear_b_p", "linear_b_g", i, j) for j in range(n)] for i in range(n)]
    ch = len(a[0][0])
    out = []
    for i in range(n):
        row = []
        for j in range(n):
            x = []
            for c in range(ch):
                s = 0.0
                for k in range(n):
                    if outgoing:
                        s += a[i][k][c] * b[j][k][c]
                    else:
                        s += a[k][i][c] * b[k][j][c]
                x.append(s)
            x = ln_vec(x, ln_out["weight"], ln_out["bias"], eps)
            y = matvec_torch(p["linear_z"]["weight"], x)
            g = matvec_torch(p["linear_g"]["weight"], zn[i][j])
            row.append([y[c] * sig(g[c]) for c in range(len(y))])
        out.append(row)
    return out


def triattn(z, mask, p, heads, starting, inf=1e9, eps=1e-5):
    """Algorithm 14/15 with torch-layout weights; softmax written out."""
    n = len(z)
    if not starting:
        z = [[z[j][i] for j in range(n)] for i in range(n)]
        mask = [[mask[j][i] for j in range(n)] for i in range(n)]
    ln = p["layer_norm"]
    att = p["attention"]
    x = [[ln_vec(z[i][j], ln["weight"], ln["bias"], eps) for j in range(n)] for i in range(n)]
    hd = len(att["linear_q"]["weight"])
    d = hd // heads
    q = [[matvec_torch(att["linear_q"]["weight"], x[i][j]) for j in range(n)] for i in range(n)]
    k = [[matvec_torch(att["linear_k"]["weight"], x[i][j]) for j in range(n)] for i in range(n)]
    v = [[matvec_torch(att["linear_v"]["weight"], x[i][j]) for j in range(n)] for i in range(n)]
    g = [[matvec_torch(att["linear_g"]["weight"], x[i][j]) for j in range(n)] for i in range(n)]
    tb = [[matvec_torch(p["linear"]["weight"], x[i][j]) for j in range(n)] for i in range(n)]
    out = [[None] * n for _ in range(n)]
    for i in range(n):
        for j in range(n):
            o = [0.0] * hd
            for h in range(heads):
                logits = []
                for kk in range(n):
                    s = sum(q[i][j][h * d + e] * k[i][kk][h * d + e] for e in range(d)) / math.sqrt(d)
                    s += inf * (mask[i][kk] - 1.0)
                    s += tb[j][kk][h]
                    logits.append(s)
                m = max(logits)
                ex = [math.exp(s - m) for s in logits]
                tot = sum(ex)
                for e in range(d):
                    acc = sum(ex[kk] / tot * v[i][kk][h * d + e] for kk in range(n))
                    o[h * d + e] = acc * sig(g[i][j][h * d + e])
            out[i][j] = matvec_torch(att["linear_o"]["weight"], o)
    if not starting:
        out = [[out[j][i] for j in range(n)] for i in range(n)]
    return out


def tolist(tree):
    if isinstance(tree, dict):
        return {k: tolist(v) for k, v in tree.items()}
    return tree.tolist()


def transition_row(x, p, eps=1e-5):
    """One row of the SwiGLU transition, written out."""
    y = ln_vec(x, p["layer_norm"]["weight"], p["layer_norm"]["bias"], eps)
    a = matvec_torch(p["linear_a"]["weight"], y)
    b = matvec_torch(p["linear_b"]["weight"], y)
    h = [a[i] * sig(a[i]) * b[i] for i in range(len(a))]
    return matvec_torch(p["linear_out"]["weight"], h)
