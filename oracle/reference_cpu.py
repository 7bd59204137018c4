"""fp32 restatement of the reference's PyTorch oracle (test infrastructure only).

Follows reference.py op for op, written independently:

* headwise (reference.py:5-20): an fp32 zero accumulator (11); taps k = 0..W-1
  in ascending order (12); the input delayed by k rows with zero fill at the
  sequence start (13); the per-head tap broadcast over the head's `D // H`
  consecutive channels (14); the static filter added to the tap, not to y
  (15-16); the residual added after the tap loop (18-19); the cast back to
  x.dtype last (20).
* lowrank (reference.py:23-39): per-token weights K = z @ U in fp32 viewed as
  [B, T, W, D] (29); + static_w (30-31); the same tap loop (34-36), residual
  (37-38) and cast (39).

Gradients are those of torch autograd through these ops, exactly as
test.py:59-69 obtains the reference gradients.

What pins these functions (tests/test_oracle.py):
  * a hand-computed known-answer case of the README formula (README.md:12-17);
  * float64 index loops and hand-derived gradient formulas (oracle/brute.py)
    on tiny shapes, including non-power-of-two head sizes and W up to 5;
  * the depthwise causal F.conv1d identity when the dynamic weight is zero;
  * W = 1 reducing to an elementwise product;
  * lowrank == headwise(hs=1) with weight = (z@U).view(B,T,W,D).transpose;
  * torch.autograd.gradcheck in float64 and the adjoint identity.
"""

import torch


def _delay(x: torch.Tensor, k: int) -> torch.Tensor:
    """Return x delayed by k rows along dim 1: out[:, t] = x[:, t-k], 0 for t < k."""
    if k == 0:
        return x
    T = x.shape[1]
    out = torch.zeros_like(x)
    if k < T:
        out[:, k:] = x[:, : T - k]
    return out


def headwise_dynamic_convolution_ref(x, weight, static_w=None, residual=False):
    """y[b,t,d] = sum_k (weight[b,t,d//hs,k] + static_w[k,d]) * x[b,t-k,d] (+ x[b,t,d]).

    Mirrors reference.py:5-20.  x [B,T,D], weight [B,T,H,W], static_w [W,D].
    Computes in float32 (or float64 when x is float64) and casts to x.dtype.
    """
    B, T, D = x.shape
    H, W = weight.shape[2], weight.shape[3]
    assert D % H == 0, f"D={D} must be divisible by H={H}"
    hs = D // H
    acc_dtype = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf = x.to(acc_dtype)
    y = torch.zeros(B, T, D, dtype=acc_dtype, device=x.device)
    for k in range(W):
        tap = weight[..., k].to(acc_dtype).repeat_interleave(hs, dim=2)  # [B,T,D]
        if static_w is not None:
            tap = tap + static_w[k].to(acc_dtype)
        y = y + tap * _delay(xf, k)
    if residual:
        y = y + xf
    return y.to(x.dtype)


def lowrank_weights_ref(z, U, D):
    """Per-token weights (z @ U).view(B, T, W, D) in fp32 (reference.py:29)."""
    B, T, R = z.shape
    W = U.shape[1] // D
    acc_dtype = torch.float64 if z.dtype == torch.float64 else torch.float32
    return (z.to(acc_dtype) @ U.to(acc_dtype)).view(B, T, W, D)


def lowrank_dynamic_convolution_ref(x, z, U, static_w=None, residual=False):
    """y[b,t,d] = sum_k ((z@U).view(B,T,W,D)[b,t,k,d] + static_w[k,d]) * x[b,t-k,d] (+ x).

    Mirrors reference.py:23-39.  x [B,T,D], z [B,T,R], U [R, W*D], static_w [W,D].
    """
    B, T, D = x.shape
    R, WD = U.shape
    assert WD % D == 0, f"Last dim. of U ({WD}) must be divisible by D={D}"
    W = WD // D
    K = lowrank_weights_ref(z, U, D)
    acc_dtype = K.dtype
    if static_w is not None:
        K = K + static_w.to(acc_dtype)
    xf = x.to(acc_dtype)
    y = torch.zeros(B, T, D, dtype=acc_dtype, device=x.device)
    for k in range(W):
        y = y + K[:, :, k, :] * _delay(xf, k)
    if residual:
        y = y + xf
    return y.to(x.dtype)
