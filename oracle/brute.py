"""float64 index-loop formulation of the hot path (test infrastructure only).

An independent restatement of README.md:12-17, used to pin
`oracle.reference_cpu` on tiny shapes.  Forward and backward are written
as explicit sums over indices, the backward from the chain rule by hand
(not from autograd), so a wrong shift direction, head mapping, tap index or
transposed operand in either formulation shows up as a mismatch.

Backward formulas (for loss L with dL/dy = dy):
  headwise
    dx[b,t,d]      = sum_k dy[b,t+k,d] * (w[b,t+k,d//hs,k] + sw[k,d])  (+ dy[b,t,d])
    dw[b,t,h,k]    = sum_{d in head h} dy[b,t,d] * x[b,t-k,d]
    dsw[k,d]       = sum_{b,t} dy[b,t,d] * x[b,t-k,d]
  lowrank (Kw[b,t,k,d] = sum_r z[b,t,r] U[r,k*D+d])
    dx[b,t,d]      = sum_k dy[b,t+k,d] * (Kw[b,t+k,k,d] + sw[k,d])  (+ dy)
    dz[b,t,r]      = sum_{k,d} dy[b,t,d] * x[b,t-k,d] * U[r,k*D+d]
    dU[r,k*D+d]    = sum_{b,t} z[b,t,r] * dy[b,t,d] * x[b,t-k,d]
    dsw[k,d]       = sum_{b,t} dy[b,t,d] * x[b,t-k,d]
with x[t] = 0 for t < 0 and dy[t] = 0 for t >= T.
"""

import numpy as np


def headwise_fwd(x, w, sw=None, residual=False):
    B, T, D = x.shape
    H, W = w.shape[2], w.shape[3]
    hs = D // H
    y = np.zeros((B, T, D), dtype=np.float64)
    for b in range(B):
        for t in range(T):
            for d in range(D):
                s = 0.0
                for k in range(W):
                    if t - k < 0:
                        continue
                    tap = w[b, t, d // hs, k] + (sw[k, d] if sw is not None else 0.0)
                    s += tap * x[b, t - k, d]
                if residual:
                    s += x[b, t, d]
                y[b, t, d] = s
    return y


def headwise_bwd(x, w, sw, dy, residual=False):
    B, T, D = x.shape
    H, W = w.shape[2], w.shape[3]
    hs = D // H
    dx = np.zeros((B, T, D))
    dw = np.zeros((B, T, H, W))
    dsw = np.zeros((W, D))
    for b in range(B):
        for t in range(T):
            for d in range(D):
                s = 0.0
                for k in range(W):
                    if t + k >= T:
                        continue
                    tap = w[b, t + k, d // hs, k] + (sw[k, d] if sw is not None else 0.0)
                    s += dy[b, t + k, d] * tap
                if residual:
                    s += dy[b, t, d]
                dx[b, t, d] = s
                for k in range(W):
                    if t - k < 0:
                        continue
                    p = dy[b, t, d] * x[b, t - k, d]
                    dw[b, t, d // hs, k] += p
                    dsw[k, d] += p
    return dx, dw, (dsw if sw is not None else None)


def lowrank_weights(z, U, D):
    B, T, R = z.shape
    W = U.shape[1] // D
    K = np.zeros((B, T, W, D))
    for b in range(B):
        for t in range(T):
            for k in range(W):
                for d in range(D):
                    K[b, t, k, d] = sum(z[b, t, r] * U[r, k * D + d] for r in range(R))
    return K


def lowrank_fwd(x, z, U, sw=None, residual=False):
    B, T, D = x.shape
    W = U.shape[1] // D
    K = lowrank_weights(z, U, D)
    y = np.zeros((B, T, D))
    for b in range(B):
        for t in range(T):
            for d in range(D):
                s = 0.0
                for k in range(W):
                    if t - k < 0:
                        continue
                    s += (K[b, t, k, d] + (sw[k, d] if sw is not None else 0.0)) * x[b, t - k, d]
                if residual:
                    s += x[b, t, d]
                y[b, t, d] = s
    return y


def lowrank_bwd(x, z, U, sw, dy, residual=False):
    B, T, D = x.shape
    R = z.shape[2]
    W = U.shape[1] // D
    K = lowrank_weights(z, U, D)
    dx = np.zeros((B, T, D))
    dz = np.zeros((B, T, R))
    dU = np.zeros_like(U, dtype=np.float64)
    dsw = np.zeros((W, D))
    for b in range(B):
        for t in range(T):
            for d in range(D):
                s = 0.0
                for k in range(W):
                    if t + k >= T:
                        continue
                    s += dy[b, t + k, d] * (K[b, t + k, k, d] + (sw[k, d] if sw is not None else 0.0))
                if residual:
                    s += dy[b, t, d]
                dx[b, t, d] = s
                for k in range(W):
                    if t - k < 0:
                        continue
                    g = dy[b, t, d] * x[b, t - k, d]
                    dsw[k, d] += g
                    for r in range(R):
                        dz[b, t, r] += g * U[r, k * D + d]
                        dU[r, k * D + d] += g * z[b, t, r]
    return dx, dz, dU, (dsw if sw is not None else None)
