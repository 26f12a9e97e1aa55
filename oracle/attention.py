"""NumPy restatements of the reference's attention oracles (oracle only).

All arrays are float32 values (bf16 / fp8 inputs already widened); outputs are
float32, the caller rounds to bf16 where the product would.  Scores are formed
in float32 by NumPy's BLAS like the reference's `Precision.HIGHEST` einsums.
"""

import math

import numpy as np

from oracle.dtypes import bf16

LOG2E = math.log2(math.e)


def fused_q_scale(softmax_scale, softcap):
    """`flywheel_tpu/softmax_attention/variant.py:80-87`: the factor folded into
    q before its bf16 rounding: softmax_scale*log2(e), or softmax_scale/softcap
    when softcap > 0 (log2(e) then applied after the tanh)."""
    if softcap == 0.0:
        return softmax_scale * LOG2E
    return softmax_scale / softcap


def _softmax_rows(scores, visible, sinks_hq):
    """Masked softmax along the last axis with optional sink logits.

    scores (..., H, Q, K) f32 natural-log logits, visible broadcastable bool,
    sinks_hq broadcastable to (..., H, Q, 1) or None.  Returns (probs, lse,
    seen) where probs excludes the sink column and rows with no visible key get
    probs 0 and lse -inf (or the sink).  Follows `util.py:233-273`.
    """
    scores = np.where(visible, scores, -np.inf)
    seen = np.broadcast_to(visible, scores.shape).any(axis=-1, keepdims=True)
    row_max = np.max(scores, axis=-1, keepdims=True, initial=-np.inf)
    if sinks_hq is not None:
        row_max = np.maximum(row_max, sinks_hq)
    anchor = np.where(np.isfinite(row_max), row_max, 0.0)
    weights = np.exp(scores - anchor)
    denom = weights.sum(axis=-1, keepdims=True)
    if sinks_hq is not None:
        denom = denom + np.exp(sinks_hq - anchor)
    probs = weights / np.where(denom > 0, denom, 1.0)
    with np.errstate(divide="ignore"):
        lse = (anchor + np.log(denom))[..., 0]
    if sinks_hq is None:
        lse = np.where(seen[..., 0], lse, -np.inf)
    probs = np.where(seen, probs, 0.0)
    return probs.astype(np.float32), lse.astype(np.float32), seen[..., 0]


def attention_ref(
    q,
    k,
    v,
    *,
    causal=False,
    window_size=(-1, -1),
    softcap=0.0,
    sinks=None,
    softmax_scale=None,
    query_lengths=None,
    key_lengths=None,
    round_scaled_q=False,
    q_chunk=512,
):
    """Naive attention, `tests/softmax_attention/util.py:181-273`.

    q (B, Sq, H, D), k / v (B, Sk, Hk, D) token-major float32.  causal and
    window_size are bottom-right aligned on each batch row's valid lengths
    (`construct_local_mask`, `util.py:148-178`): query i of a row with lengths
    (sq, sk) sits on diagonal i + sk - sq; causal forces the right bound to 0.
    softcap > 0 maps each scaled score s to tanh(s/softcap)*softcap before the
    mask.  sinks (H,) join each head's softmax with no value row.
    round_scaled_q rounds q*fused_q_scale to bf16 first, as every kernel of
    the path does (`decode.py:517-520`, `variant.py:transform_q`).

    Returns (out (B, Sq, H, D) f32, lse (B, H, Sq) f32).  Padded queries and
    rows with no visible key get out 0; lse -inf on those rows (or the sink).
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    batch, seqlen_q, nheads, head_dim = q.shape
    seqlen_k, nheads_k = k.shape[1], k.shape[2]
    group = nheads // nheads_k
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    left, right = window_size
    if causal:
        right = 0
    qlens = np.full(batch, seqlen_q) if query_lengths is None else np.asarray(query_lengths)
    klens = np.full(batch, seqlen_k) if key_lengths is None else np.asarray(key_lengths)
    out = np.zeros((batch, seqlen_q, nheads, v.shape[-1]), np.float32)
    lse = np.full((batch, nheads, seqlen_q), -np.inf, np.float32)
    sinks_h = None if sinks is None else np.asarray(sinks, np.float32)
    for b in range(batch):
        kb = np.repeat(k[b], group, axis=1).transpose(1, 2, 0)  # (H, D, Sk)
        vb = np.repeat(v[b], group, axis=1).transpose(1, 0, 2)  # (H, Sk, D)
        cols = np.arange(seqlen_k)[None, :]
        for c0 in range(0, seqlen_q, q_chunk):
            rows = np.arange(c0, min(c0 + q_chunk, seqlen_q))
            qb = q[b, rows].transpose(1, 0, 2)  # (H, Q, D)
            if round_scaled_q:
                qs = bf16(qb * np.float32(fused_q_scale(scale, softcap)))
                raw = qs @ kb
                if softcap > 0:
                    scores = np.tanh(raw) * np.float32(softcap)
                else:
                    scores = raw * np.float32(math.log(2.0))
            else:
                scores = (qb * np.float32(scale)) @ kb
                if softcap > 0:
                    scores = np.tanh(scores / np.float32(softcap)) * np.float32(softcap)
            diagonal = rows[:, None] + klens[b] - qlens[b]
            visible = cols < klens[b]
            if right >= 0:
                visible = visible & (cols <= diagonal + right)
            if left >= 0:
                visible = visible & (cols >= diagonal - left)
            visible = visible & (rows[:, None] < qlens[b])
            sk = None if sinks_h is None else sinks_h[:, None, None]
            probs, row_lse, _ = _softmax_rows(scores, visible[None], sk)
            ob = probs @ vb  # (H, Q, D)
            out[b, rows] = ob.transpose(1, 0, 2)
            valid_q = rows < qlens[b]
            out[b, rows[~valid_q]] = 0.0
            lse[b, :, rows] = row_lse.T
            if sinks_h is None:
                lse[b, :, rows[~valid_q]] = -np.inf
    return out, lse


def kvcache_reference(
    q,
    k_rows,
    v_rows,
    total_lengths,
    *,
    causal=False,
    window_size=(-1, -1),
    softcap=0.0,
    sinks=None,
    softmax_scale=None,
    k_descale=1.0,
    v_descale=1.0,
    round_scaled_q=True,
):
    """One flash_attn_with_kvcache step over gathered cache rows.

    Restates `decode_reference` (`tests/softmax_attention/test_regression.py:
    901-961`) generalised to seqlen_q >= 1 query tokens per row (the folded
    verify window, `kernels/decode.py:560-575`): token t of row b sits at
    position total_lengths[b] - seqlen_q + t.

    q (B, Sq, H, D) f32; k_rows / v_rows (B, cap, Hk, D) f32 *stored* values
    (fp8 codes widened, not yet descaled).  Following `decode.py:512-520` the
    scores start from bf16(q * fused_q_scale(scale * k_descale, softcap)); the
    output is multiplied by v_descale (`variant.py:352-363`).
    Returns (out (B, Sq, H, D) f32, lse (B, H, Sq) f32).
    """
    q = np.asarray(q, np.float32)
    batch, seqlen_q, nheads, head_dim = q.shape
    cap, nheads_k = k_rows.shape[1], k_rows.shape[2]
    group = nheads // nheads_k
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    qscale = fused_q_scale(scale * float(k_descale), softcap)
    q_scaled = bf16(q * np.float32(qscale)) if round_scaled_q else q * np.float32(qscale)
    left, right = window_size
    if causal:
        right = 0
    out = np.zeros((batch, seqlen_q, nheads, head_dim), np.float32)
    lse = np.full((batch, nheads, seqlen_q), -np.inf, np.float32)
    sinks_h = None if sinks is None else np.asarray(sinks, np.float32)[:, None, None]
    keys_pos = np.arange(cap)[None, :]
    for b in range(batch):
        total = int(total_lengths[b])
        kb = np.repeat(np.asarray(k_rows[b], np.float32), group, axis=1).transpose(1, 2, 0)
        vb = np.repeat(np.asarray(v_rows[b], np.float32), group, axis=1).transpose(1, 0, 2)
        qb = q_scaled[b].transpose(1, 0, 2)  # (H, Sq, D)
        raw = qb @ kb  # (H, Sq, cap)
        if softcap > 0:
            scores = np.tanh(raw) * np.float32(softcap)
        else:
            scores = raw * np.float32(math.log(2.0))
        qpos = (total - seqlen_q + np.arange(seqlen_q))[:, None]
        visible = keys_pos < total
        if right >= 0:
            visible = visible & (keys_pos <= qpos + right)
        if left >= 0:
            visible = visible & (keys_pos >= qpos - left)
        probs, row_lse, _ = _softmax_rows(scores, visible[None], sinks_h)
        ob = probs @ vb * np.float32(v_descale)
        out[b] = ob.transpose(1, 0, 2)
        lse[b] = row_lse
    return out, lse


def decode_reference(q, k_cache, v_cache, cache_seqlens, cache_batch_idx=None, **kwargs):
    """`test_regression.py:901-961`: the single-token form of kvcache_reference
    over contiguous caches mapped by cache_batch_idx."""
    if cache_batch_idx is None:
        cache_batch_idx = np.arange(q.shape[0])
    return kvcache_reference(
        q, k_cache[cache_batch_idx], v_cache[cache_batch_idx], cache_seqlens, **kwargs
    )


def ragged_reference(
    q,
    k_pages,
    v_pages,
    cu_seqlens_q,
    seqused_k,
    table,
    *,
    causal,
    window_left=None,
    softcap=0.0,
    sinks=None,
    softmax_scale=None,
    k_descale=1.0,
    v_descale=1.0,
    round_scaled_q=False,
    num_active=None,
):
    """Packed rows attending a paged cache, `test_paged.py:98-206`.

    q (T, H, D) f32 packed by cu_seqlens_q; k_pages / v_pages (pages, P, Hk, D)
    f32 stored values (the caller appends new tokens first, see
    `paged.append_to_pages`).  seqused_k[s] is the sequence's kv length with its
    new tokens.  Row i of sequence s sits on diagonal seqused_k[s] - len_q + i;
    causal hides keys past it; window_left hides keys more than window_left
    before it.  Rows past cu_seqlens_q[num_active] are padding: out 0, lse -inf.
    Returns (out (T, H, D) f32, lse (H, T) f32).
    """
    q = np.asarray(q, np.float32)
    total_q, nheads, head_dim = q.shape
    page_size, nheads_k = k_pages.shape[1], k_pages.shape[2]
    group = nheads // nheads_k
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    qscale = np.float32(scale * float(k_descale))
    cu = np.asarray(cu_seqlens_q)
    lens = np.asarray(seqused_k)
    table = np.asarray(table)
    batch = len(cu) - 1
    if num_active is not None:
        batch = int(num_active)
    out = np.zeros_like(q)
    lse = np.full((nheads, total_q), -np.inf, np.float32)
    sinks_h = None if sinks is None else np.asarray(sinks, np.float32)[:, None, None]
    for s in range(batch):
        start, end = int(cu[s]), int(cu[s + 1])
        qlen = end - start
        if qlen <= 0:
            continue
        total = int(lens[s])
        positions = np.arange(total)
        pages = table[s, positions // page_size]
        keys = np.asarray(k_pages[pages, positions % page_size], np.float32)  # (L, Hk, D)
        vals = np.asarray(v_pages[pages, positions % page_size], np.float32)
        kb = np.repeat(keys, group, axis=1).transpose(1, 2, 0)  # (H, D, L)
        vb = np.repeat(vals, group, axis=1).transpose(1, 0, 2)  # (H, L, D)
        for c0 in range(0, qlen, 256):
            rows = np.arange(c0, min(c0 + 256, qlen))
            qb = q[start + rows].transpose(1, 0, 2)
            if round_scaled_q:
                qs = bf16(qb * np.float32(fused_q_scale(float(qscale), softcap)))
                raw = qs @ kb
                scores = (np.tanh(raw) * np.float32(softcap)) if softcap > 0 else raw * np.float32(math.log(2.0))
            else:
                scores = (qb * qscale) @ kb
                if softcap > 0:
                    scores = np.float32(softcap) * np.tanh(scores / np.float32(softcap))
            diagonal = (total - qlen + rows)[:, None]
            visible = np.ones((len(rows), total), bool)
            if causal:
                visible &= positions[None] <= diagonal
            if window_left is not None and window_left >= 0:
                visible &= positions[None] >= diagonal - window_left
            probs, row_lse, _ = _softmax_rows(scores, visible[None], sinks_h)
            ob = probs @ vb * np.float32(v_descale)
            out[start + rows] = ob.transpose(1, 0, 2)
            lse[:, start + rows] = row_lse
    return out, lse
