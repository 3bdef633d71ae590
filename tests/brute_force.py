"""Float64 scalar-loop formulations used to pin ``oracle.reference``.

Written from the algorithm definitions (AlphaFold2 supplement Alg. 11-14,
AlphaFold3 Alg. 17/24/11 as implemented by the reference), one output element
at a time with explicit loops over every index, so that a dropped term, a
swapped index or a transposed operand in the vectorised oracle shows up as a
mismatch.  Tiny shapes only (N <= ~8).
"""

from __future__ import annotations

import math

import numpy as np

EPS = 1e-5
INF = 1e9


def _np(t):
    return t.detach().cpu().double().numpy() if hasattr(t, "detach") else np.asarray(t, np.float64)


def ln_vec(x, w, b):
    n = len(x)
    mu = sum(x) / n
    var = sum((xi - mu) ** 2 for xi in x) / n
    r = 1.0 / math.sqrt(var + EPS)
    return [((x[c] - mu) * r) * (w[c] if w is not None else 1.0) + (b[c] if b is not None else 0.0)
            for c in range(n)]


def matvec(W, x):
    """y[o] = sum_c W[o][c] x[c]."""
    return [sum(W[o][c] * x[c] for c in range(len(x))) for o in range(len(W))]


def sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def layer_norm_rows(x, w, b):
    x = _np(x)
    out = np.zeros_like(x)
    flat = x.reshape(-1, x.shape[-1])
    of = out.reshape(-1, x.shape[-1])
    for r in range(flat.shape[0]):
        of[r] = ln_vec(list(flat[r]), None if w is None else list(_np(w)),
                       None if b is None else list(_np(b)))
    return out


def layer_norm_backward_rows(x, w, dout):
    """grad_input[r][c] = sum_o dout[r][o] * d ln(x[r])[o] / d x[r][c] and
    grad_w[c] = sum_r dout[r][c] * xhat[r][c], grad_b[c] = sum_r dout[r][c],
    from the derivative of LN written out element by element:
        xhat_o = (x_o - mu) r,   r = (var + eps)^(-1/2)
        d xhat_o / d x_c = r (delta_oc - 1/n) - xhat_o xhat_c r / n."""
    x, dout = _np(x), _np(dout)
    n = x.shape[-1]
    xf, df = x.reshape(-1, n), dout.reshape(-1, n)
    wv = [1.0] * n if w is None else list(_np(w))
    gi = np.zeros_like(xf)
    gw = np.zeros(n)
    gb = np.zeros(n)
    for r in range(xf.shape[0]):
        row = list(xf[r])
        mu = sum(row) / n
        var = sum((v - mu) ** 2 for v in row) / n
        rs = 1.0 / math.sqrt(var + EPS)
        xh = [(v - mu) * rs for v in row]
        for c in range(n):
            acc = 0.0
            for o in range(n):
                dxh = rs * ((1.0 if o == c else 0.0) - 1.0 / n) - xh[o] * xh[c] * rs / n
                acc += df[r][o] * wv[o] * dxh
            gi[r][c] = acc
            gw[c] += df[r][c] * xh[c]
            gb[c] += df[r][c]
    return gi.reshape(x.shape), gw, gb


def triangle_attention(z, mask, p, H, starting=True):
    """Alg. 13 (starting node), for every (i, j) and head h:
        a[k] = softmax_k( q_h[i,j].k_h[i,k]/sqrt(D) + b_h[j,k] + INF*(mask[i,k]-1) )
        out[i,j] = W_o( concat_h sigmoid(g_h[i,j]) * sum_k a[k] v_h[i,k] )
    Alg. 14 (ending node), written with its own indices (no transposes):
        a[k] = softmax_k( q_h[i,j].k_h[k,j]/sqrt(D) + b_h[k,i] + INF*(mask[k,j]-1) )
        out[i,j] = W_o( concat_h sigmoid(g_h[i,j]) * sum_k a[k] v_h[k,j] )
    where every per-position quantity is computed from x = LN(z) at that
    position."""
    z = _np(z)
    N = z.shape[0]
    mask = np.ones((N, N)) if mask is None else _np(mask)
    P = {k: _np(v) for k, v in p.items()}
    HD = P["mha.linear_q.weight"].shape[0]
    D = HD // H
    x = [[ln_vec(list(z[i, j]), P["layer_norm.weight"], P["layer_norm.bias"])
          for j in range(N)] for i in range(N)]
    q = [[matvec(P["mha.linear_q.weight"], x[i][j]) for j in range(N)] for i in range(N)]
    k = [[matvec(P["mha.linear_k.weight"], x[i][j]) for j in range(N)] for i in range(N)]
    v = [[matvec(P["mha.linear_v.weight"], x[i][j]) for j in range(N)] for i in range(N)]
    g = [[matvec(P["mha.linear_g.weight"], x[i][j]) for j in range(N)] for i in range(N)]
    tb = [[matvec(P["linear.weight"], x[i][j]) for j in range(N)] for i in range(N)]
    out = np.zeros((N, N, z.shape[2]))
    for i in range(N):
        for j in range(N):
            o = [0.0] * HD
            for h in range(H):
                logits = []
                for kk in range(N):
                    if starting:
                        kv_pos, b_pos, m_pos = (i, kk), (j, kk), (i, kk)
                    else:
                        kv_pos, b_pos, m_pos = (kk, j), (kk, i), (kk, j)
                    kvec = k[kv_pos[0]][kv_pos[1]]
                    s = sum(q[i][j][h * D + d] * kvec[h * D + d] for d in range(D)) / math.sqrt(D)
                    s += INF * (mask[m_pos] - 1.0)
                    s += tb[b_pos[0]][b_pos[1]][h]
                    logits.append(s)
                mx = max(logits)
                e = [math.exp(t - mx) for t in logits]
                den = sum(e)
                for d in range(D):
                    acc = 0.0
                    for kk in range(N):
                        vv = v[i][kk] if starting else v[kk][j]
                        acc += e[kk] / den * vv[h * D + d]
                    o[h * D + d] = acc * sigmoid(g[i][j][h * D + d])
            out[i, j] = matvec(P["mha.linear_o.weight"], o)
    return out


def triangle_multiplication(z, mask, p, outgoing=True):
    """Alg. 11/12: x = LN(z); a = m*sig(Wag x)*(Wap x); b likewise;
    outgoing p[i,j] = sum_k a[i,k]*b[j,k]; incoming p[i,j] = sum_k a[k,i]*b[k,j];
    out[i,j] = sig(Wg x[i,j]) * Wz LN(p[i,j])."""
    z = _np(z)
    N = z.shape[0]
    mask = np.ones((N, N)) if mask is None else _np(mask)
    P = {k: _np(v) for k, v in p.items()}
    x = [[ln_vec(list(z[i, j]), P["layer_norm_in.weight"], P["layer_norm_in.bias"])
          for j in range(N)] for i in range(N)]
    Ch = P["linear_a_p.weight"].shape[0]

    def proj(w_g, w_p, i, j):
        gg = matvec(P[w_g], x[i][j])
        pp = matvec(P[w_p], x[i][j])
        return [mask[i, j] * sigmoid(gg[c]) * pp[c] for c in range(Ch)]
    a = [[proj("linear_a_g.weight", "linear_a_p.weight", i, j) for j in range(N)] for i in range(N)]
    b = [[proj("linear_b_g.weight", "linear_b_p.weight", i, j) for j in range(N)] for i in range(N)]
    out = np.zeros_like(z)
    for i in range(N):
        for j in range(N):
            pij = []
            for c in range(Ch):
                if outgoing:
                    pij.append(sum(a[i][kk][c] * b[j][kk][c] for kk in range(N)))
                else:
                    pij.append(sum(a[kk][i][c] * b[kk][j][c] for kk in range(N)))
            y = matvec(P["linear_z.weight"],
                       ln_vec(pij, P["layer_norm_out.weight"], P["layer_norm_out.bias"]))
            gg = matvec(P["linear_g.weight"], x[i][j])
            out[i, j] = [y[c] * sigmoid(gg[c]) for c in range(len(y))]
    return out


def contract(a, b, outgoing=True):
    """p[i,j,c] triple loop."""
    a, b = _np(a), _np(b)
    N, _, C = a.shape
    out = np.zeros((N, N, C))
    for i in range(N):
        for j in range(N):
            for c in range(C):
                if outgoing:
                    out[i, j, c] = sum(a[i, kk, c] * b[j, kk, c] for kk in range(N))
                else:
                    out[i, j, c] = sum(a[kk, i, c] * b[kk, j, c] for kk in range(N))
    return out


def transition(x, p):
    """Alg. 11 (AF3): y = LN(x); out = Wo( silu(Wa y) * (Wb y) )."""
    x = _np(x)
    P = {k: _np(v) for k, v in p.items()}
    flat = x.reshape(-1, x.shape[-1])
    out = np.zeros((flat.shape[0], P["linear_no_bias.weight"].shape[0]))
    for r in range(flat.shape[0]):
        y = ln_vec(list(flat[r]), P["layernorm1.weight"], P["layernorm1.bias"])
        a = matvec(P["linear_no_bias_a.weight"], y)
        bb = matvec(P["linear_no_bias_b.weight"], y)
        h = [a[t] * sigmoid(a[t]) * bb[t] for t in range(len(a))]
        out[r] = matvec(P["linear_no_bias.weight"], h)
    return out.reshape(x.shape[:-1] + (out.shape[-1],))


def outer_product_mean(m, mask, p, eps=1e-3):
    """Alg. 9 (AF3) / Alg. 10 (AF2) OuterProductMean, one output element at a
    time: y[s,i] = LN(m[s,i]); a[s,i,c] = mask[s,i] (W1 y[s,i])[c] (+ b1);
    b likewise; o[i,j,c1,c2] = sum_s a[s,i,c1] b[s,j,c2];
    out[i,j,z] = (sum_{c1,c2} Wout[z][c1*C+c2] o[i,j,c1,c2] + bout[z])
                 / (sum_s mask[s,i] mask[s,j] + eps)."""
    m = _np(m)
    S, N, _ = m.shape
    mk = np.ones((S, N)) if mask is None else _np(mask)
    P = {k: _np(v) for k, v in p.items()}
    W1, W2, Wo = P["linear_1.weight"], P["linear_2.weight"], P["linear_out.weight"]
    C = W1.shape[0]
    a = np.zeros((S, N, C))
    b = np.zeros((S, N, C))
    for s in range(S):
        for i in range(N):
            y = ln_vec(list(m[s, i]), P["layer_norm.weight"], P["layer_norm.bias"])
            av, bv = matvec(W1, y), matvec(W2, y)
            for c in range(C):
                a[s, i, c] = mk[s, i] * (av[c] + (P["linear_1.bias"][c] if "linear_1.bias" in P else 0.0))
                b[s, i, c] = mk[s, i] * (bv[c] + (P["linear_2.bias"][c] if "linear_2.bias" in P else 0.0))
    out = np.zeros((N, N, Wo.shape[0]))
    for i in range(N):
        for j in range(N):
            norm = sum(mk[s, i] * mk[s, j] for s in range(S)) + eps
            for zc in range(Wo.shape[0]):
                acc = 0.0
                for c1 in range(C):
                    for c2 in range(C):
                        o = sum(a[s, i, c1] * b[s, j, c2] for s in range(S))
                        acc += Wo[zc][c1 * C + c2] * o
                if "linear_out.bias" in P:
                    acc += P["linear_out.bias"][zc]
                out[i, j, zc] = acc / norm
    return out


def attention_pair_bias(s, z, p, n_heads):
    """Alg. 24 (has_s=False): a = LN(s); bias_h[i,j] = Wz LN(z[i,j]);
    out[i] = Wo( concat_h sig(Wg a[i]) * softmax_j(q_h[i].k_h[j]/sqrt(dh) + bias_h[i,j]) v_h[j] ),
    q = Wq a + bq."""
    s, z = _np(s), _np(z)
    P = {k: _np(v) for k, v in p.items()}
    N, c_a = s.shape
    dh = c_a // n_heads
    a = [ln_vec(list(s[i]), P["layernorm_a.weight"], P["layernorm_a.bias"]) for i in range(N)]
    bias = [[matvec(P["linear_nobias_z.weight"],
                    ln_vec(list(z[i, j]), P["layernorm_z.weight"], P["layernorm_z.bias"]))
             for j in range(N)] for i in range(N)]
    q = [[t + bq for t, bq in zip(matvec(P["attention.linear_q.weight"], a[i]),
                                  P["attention.linear_q.bias"])] for i in range(N)]
    k = [matvec(P["attention.linear_k.weight"], a[i]) for i in range(N)]
    v = [matvec(P["attention.linear_v.weight"], a[i]) for i in range(N)]
    g = [matvec(P["attention.linear_g.weight"], a[i]) for i in range(N)]
    out = np.zeros((N, P["attention.linear_o.weight"].shape[0]))
    for i in range(N):
        o = [0.0] * c_a
        for h in range(n_heads):
            logits = [sum(q[i][h * dh + d] * k[j][h * dh + d] for d in range(dh)) / math.sqrt(dh)
                      + bias[i][j][h] for j in range(N)]
            mx = max(logits)
            e = [math.exp(t - mx) for t in logits]
            den = sum(e)
            for d in range(dh):
                o[h * dh + d] = sum(e[j] / den * v[j][h * dh + d] for j in range(N)) \
                    * sigmoid(g[i][h * dh + d])
        out[i] = matvec(P["attention.linear_o.weight"], o)
    return out


def _sub(p, prefix):
    return {k[len(prefix):]: v for k, v in p.items() if k.startswith(prefix)}


def pairformer_block(s, z, mask, p, H, n_heads):
    """Alg. 17 block in the reference's order, residual after every member."""
    z = _np(z).copy()
    mask = _np(mask)
    z = z + triangle_multiplication(z, mask, _sub(p, "tri_mul_out."), True)
    z = z + triangle_multiplication(z, mask, _sub(p, "tri_mul_in."), False)
    z = z + triangle_attention(z, mask, _sub(p, "tri_att_start."), H, True)
    z = z + triangle_attention(z, mask, _sub(p, "tri_att_end."), H, False)
    z = z + transition(z, _sub(p, "pair_transition."))
    if s is not None:
        s = _np(s)
        s = s + attention_pair_bias(s, z, _sub(p, "attention_pair_bias."), n_heads)
        s = s + transition(s, _sub(p, "single_transition."))
    return s, z
