"""numpy fp64 restatement of the dense hot path.  TEST INFRASTRUCTURE ONLY.

gemm                 C = A @ B                          GEMMKernel.swift:28-174; DotTests.swift:16-30
attention_forward    O, P, L (log2 units)               AttentionTests.swift:21-54;
                                                        attention_training.py:170-176;
                                                        AttentionKernel.swift:33-39 (L = m + log2 l)
attention_backward   Delta, dQ, dK, dV, amplification   AttentionBackwardTests.swift:46-160;
                                                        attention_training.py:179-187
attention_head_f32   one head's fwd + bwd via BLAS        attention_training.py:170-187
attention_head_causal_blocked_f32  the same, causal, by query-row blocks over visible keys only
                                                        (the CPU baseline)
sae_encode           relu(x @ W_enc + b_enc)            SAEEncoder.swift:1-20;
                                                        sae_encode.py:60-61 (numpy reference)
The causal mask (key j > query i excluded) is this build's extension; the
reference has none.  Arrays are [heads, seq, dim].
"""

import functools
import math

import numpy as np

LOG2E = 1.4426950408889634


def gemm(a, b) -> np.ndarray:
    return np.asarray(a, np.float64) @ np.asarray(b, np.float64)


def sae_encode(x, w, b) -> np.ndarray:
    """relu(x @ w + b) in fp64: the fused SAE encoder's definition."""
    return np.maximum(gemm(x, w) + np.asarray(b, np.float64)[None, :], 0.0)


def _scores(q, k, scale, causal):
    s = np.einsum("hid,hjd->hij", q, k) * scale
    if causal:
        n = s.shape[-1]
        mask = np.triu(np.ones((n, n), dtype=bool), 1)
        s = np.where(mask[None], -np.inf, s)
    return s


def attention_forward(q, k, v, scale, causal=False):
    """fp64 stable softmax attention.  Returns (O, P, L) with L = log2 of the
    unshifted softmax denominator, exactly what attn_fwd writes."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    s = _scores(q, k, scale, causal)
    peak = s.max(axis=-1, keepdims=True)
    e = np.exp(s - peak)
    total = e.sum(axis=-1, keepdims=True)
    p = e / total
    o = np.einsum("hij,hjd->hid", p, v)
    lse2 = (peak[..., 0] * LOG2E) + np.log2(total[..., 0])
    return o, p, lse2


def attention_backward(q, k, v, d_out, scale, causal=False):
    """fp64 analytic gradients from the definitions, plus the reference's
    cancellation amplification A = max_i sum_j |term_ij| / max|grad|."""
    q, k, v, d_out = (np.asarray(x, np.float64) for x in (q, k, v, d_out))
    o, p, lse2 = attention_forward(q, k, v, scale, causal)
    delta = np.einsum("hid,hid->hi", d_out, o)
    dp = np.einsum("hid,hjd->hij", d_out, v)
    ds = p * (dp - delta[..., None])
    dq = np.einsum("hij,hjd->hid", ds, k) * scale
    dk = np.einsum("hij,hid->hjd", ds, q) * scale
    dv = np.einsum("hij,hid->hjd", p, d_out)

    def amp(terms_abs_sum, grad):
        return float(terms_abs_sum.max() / max(np.abs(grad).max(), 1e-30))

    amplification = {
        "dq": amp(np.einsum("hij,hjd->hid", np.abs(ds), np.abs(k)) * scale, dq),
        "dk": amp(np.einsum("hij,hid->hjd", np.abs(ds), np.abs(q)) * scale, dk),
        "dv": amp(np.einsum("hij,hid->hjd", p, np.abs(d_out)), dv),
    }
    return {"o": o, "p": p, "lse": lse2, "delta": delta, "dq": dq, "dk": dk, "dv": dv,
            "amplification": amplification}


def loss_o_dot_do(q, k, v, d_out, scale, causal=False) -> float:
    """sum(O * dO): its gradient w.r.t. Q, K, V is exactly (dQ, dK, dV) for
    upstream gradient dO (AttentionBackwardTests.swift:162-197)."""
    o, _, _ = attention_forward(q, k, v, scale, causal)
    return float(np.sum(o * np.asarray(d_out, np.float64)))


def finite_difference(q, k, v, d_out, scale, which, index, h=1e-5, causal=False) -> float:
    """Central difference of sum(O*dO) w.r.t. one element of Q, K or V."""
    args = [np.array(x, np.float64) for x in (q, k, v)]
    slot = {"dq": 0, "dk": 1, "dv": 2}[which]
    plus = [a.copy() for a in args]
    minus = [a.copy() for a in args]
    plus[slot][index] += h
    minus[slot][index] -= h
    return (loss_o_dot_do(*plus, d_out, scale, causal)
            - loss_o_dot_do(*minus, d_out, scale, causal)) / (2 * h)


def numpy_attention_f32(q, k, v, scale):
    """The reference's float32 numpy forward, restated (attention_training.py:170-176):
    the same arithmetic in the same dtype, for reproducing its published run."""
    scores = np.einsum("hid,hjd->hij", q, k) * scale
    scores = scores - scores.max(axis=-1, keepdims=True)
    weights = np.exp(scores)
    weights = weights / weights.sum(axis=-1, keepdims=True)
    return np.einsum("hij,hjd->hid", weights, v), weights


def numpy_attention_backward_f32(q, k, v, weights, d_out, scale):
    """attention_training.py:179-187, restated."""
    dv = np.einsum("hij,hid->hjd", weights, d_out)
    dp = np.einsum("hid,hjd->hij", d_out, v)
    delta = (dp * weights).sum(axis=-1, keepdims=True)
    ds = weights * (dp - delta)
    dq = np.einsum("hij,hjd->hid", ds, k) * scale
    dk = np.einsum("hij,hid->hjd", ds, q) * scale
    return dq, dk, dv


@functools.lru_cache(maxsize=4)
def _causal_bias(rows, cols):
    """float32 [rows, cols]: 0 where key j <= query i, -inf above the diagonal."""
    bias = np.zeros((rows, cols), np.float32)
    bias[np.triu_indices(rows, 1, cols)] = -np.inf
    return bias


def attention_head_f32(q, k, v, d_out, scale, causal=False):
    """One head's forward and backward in float32 through BLAS matmuls: the
    arithmetic of numpy_attention_f32 and numpy_attention_backward_f32
    (attention_training.py:170-187) with `@` in place of einsum and Delta as
    rowsum(dO * O), plus the causal mask (keys after the query excluded).  [S, D] inputs; returns
    (O, dQ, dK, dV).  This is what the benchmark's CPU baseline times."""
    scale = np.float32(scale)
    s = (q @ k.T) * scale
    if causal:
        s += _causal_bias(s.shape[0], s.shape[1])
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    o = p @ v
    dv = p.T @ d_out
    dp = d_out @ v.T
    # rowsum(dP * P) as the reference writes it equals rowsum(dO * O), an [S, D]
    # product instead of an [S, S] one (the FlashAttention-2 Delta)
    delta = (d_out * o).sum(-1, keepdims=True)
    ds = p * (dp - delta)
    dq = (ds @ k) * scale
    dk = (ds.T @ q) * scale
    return o, dq, dk, dv


def attention_head_causal_blocked_f32(q, k, v, d_out, scale, block=512):
    """attention_head_f32 with causal=True, computed one block of `block` query
    rows at a time over only the keys those rows can see (keys 0 .. the
    block's last row): the same float32 BLAS arithmetic row by row (each row's
    softmax still sees its whole visible key range at once), without the
    masked upper triangle's work beyond the diagonal blocks.  At S = 4096 and
    block 512 it executes 36/64 of the full S^2 products (the causal half plus
    the diagonal blocks).  [S, D] inputs; returns (O, dQ, dK, dV).  This is what
    the benchmark's CPU baseline times."""
    scale = np.float32(scale)
    n = q.shape[0]
    o = np.empty_like(q)
    dq = np.empty_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for r0 in range(0, n, block):
        r1 = min(n, r0 + block)
        kv = r1  # keys 0 .. r1-1 are visible to some row of the block
        s = (q[r0:r1] @ k[:kv].T) * scale
        s += _causal_bias(n, n)[r0:r1, :kv]
        s -= s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        o[r0:r1] = p @ v[:kv]
        dv[:kv] += p.T @ d_out[r0:r1]
        dp = d_out[r0:r1] @ v[:kv].T
        delta = (d_out[r0:r1] * o[r0:r1]).sum(-1, keepdims=True)
        ds = p * (dp - delta)
        dq[r0:r1] = (ds @ k[:kv]) * scale
        dk[:kv] += (ds.T @ q[r0:r1]) * scale
    return o, dq, dk, dv


def reference_training_inputs(heads=2, seq=96, dim=64, seed=0, spread=0.5):
    """The published attention training run's inputs (attention_training.py:256-261):
    default_rng(0), q, k, v, target = standard_normal(float32) * 0.5, in that order."""
    rng = np.random.default_rng(seed)
    shape = (heads, seq, dim)
    q = rng.standard_normal(shape, dtype=np.float32) * spread
    k = rng.standard_normal(shape, dtype=np.float32) * spread
    v = rng.standard_normal(shape, dtype=np.float32) * spread
    target = rng.standard_normal(shape, dtype=np.float32) * spread
    return q, k, v, target


def training_run(grad_fn, forward_fn, q, k, v, target, rate, steps=8):
    """Gradient descent on 0.5*||O - T||^2 (attention_training.py:312-329).
    grad_fn(q, k, v, d_out) -> (dq, dk, dv); forward_fn(q, k, v) -> O.
    Returns the per-step records and the final loss."""
    records = []
    for _ in range(steps):
        out = forward_fn(q, k, v)
        loss = 0.5 * float(np.sum((out.astype(np.float64) - target) ** 2))
        d_out = (out - target).astype(np.float32)
        dq, dk, dv = grad_fn(q, k, v, d_out)
        records.append({"loss": loss, "dq": float(np.linalg.norm(dq)),
                        "dk": float(np.linalg.norm(dk)), "dv": float(np.linalg.norm(dv))})
        q = (q - rate * dq).astype(np.float32)
        k = (k - rate * dk).astype(np.float32)
        v = (v - rate * dv).astype(np.float32)
    final = 0.5 * float(np.sum((forward_fn(q, k, v).astype(np.float64) - target) ** 2))
    return records, final


def attention_flops(batch_heads, seq, dim, causal, backward=False) -> float:
    """The reference's FLOP convention: 4*S^2*D forward, 10*S^2*D backward per
    (batch*head) (AttentionBenchmark.swift:64-68, AttentionBackwardBenchmark.swift:45-49);
    causal counts half (this build's convention)."""
    per = (10.0 if backward else 4.0) * seq * seq * dim * batch_heads
    return per / 2 if causal else per


def gemm_flops(m, n, k) -> float:
    """2*M*N*K (GEMMBenchmark.swift:449-451)."""
    return 2.0 * m * n * k


def sqrt_scale(dim):
    return 1.0 / math.sqrt(dim)
