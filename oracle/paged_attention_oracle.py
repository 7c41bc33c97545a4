"""CPU oracle for the paged-attention path (KV store, block-table gather,
ragged causal GQA prefill, split-K decode).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use it, and only to check results.  The HIP path never
falls back to it.

Every function restates, in numpy, the algorithm of the reference file:line
it cites (simpissa/vllm-jax).  The reference is JAX/Pallas code that lowers to
Triton; it cannot run in this environment (no JAX, Python 3.10), so the
restatement is pinned by closed forms, brute force and invariants in
``tests/test_oracle.py``:

* ``kv_store``      -- closed form ``pool'[slot[t]] == k[t]``, all other slots
                       untouched (bit-exact).
* ``gather_kv``     -- closed form ``ctx[b, j] == pool[bt[b, j // BS], j % BS]``.
* ``prefill_attention`` / ``decode_attention`` -- float64 brute force
  (``dense_*_f64``), context-length-1 => ``v_0``, equal keys => mean(v),
  length 0 => 0, block relabelling invariance, split-count invariance,
  prefix truncation, prefill-last-row == decode.

bf16 values are carried as ``uint16`` bit patterns; arithmetic is float32 with
explicit round-to-nearest-even bf16 rounding wherever the reference stores a
bf16 intermediate.
"""
from __future__ import annotations

import math

import numpy as np

# prefill_paged_attention.py:15 / decode_paged_attention.py:31
DEFAULT_MASK_VALUE = -0.7 * float(np.finfo(np.float32).max)
F32_MIN = float(np.finfo(np.float32).min)
F32_EPS = float(np.finfo(np.float32).eps)
LOG2E = math.log2(math.e)


# ----------------------------------------------------------------------------
# bf16 helpers
# ----------------------------------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round to nearest even; NaN kept."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_to_f32(b) -> np.ndarray:
    """bf16 bit pattern (uint16) -> float32 (exact)."""
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """Round float32 values through bf16 and back (the value a bf16 store keeps)."""
    return bf16_to_f32(f32_to_bf16(x))


def _as_f32(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return bf16_to_f32(a)
    return a.astype(np.float32)


# ----------------------------------------------------------------------------
# a2: KV store  (qwen3.py:105-111)
# ----------------------------------------------------------------------------
def kv_store(k_cache, v_cache, k, v, slot_mapping):
    """Scatter new K/V token rows into the paged pool.

    Restates ``_update_kv_cache`` (vllm/model/qwen3.py:105-111): the pool
    ``[NB, BS, Hkv, d]`` is viewed as ``[NB*BS, Hkv, d]`` and
    ``flat[slot[t]] = k[t]`` (same for v).  ``mode="drop"`` drops slots past
    the end (qwen3.py:109-110).  Slots < 0 mark padding tokens
    (model_runner.py:249,292) and are skipped (the reference's evident intent;
    JAX would wrap -1 to the last slot, see the contract note in the tests).

    Returns new (k_cache, v_cache) arrays; inputs are not modified.
    """
    k_cache = np.array(k_cache, copy=True)
    v_cache = np.array(v_cache, copy=True)
    nb, bs, hkv, d = k_cache.shape
    fk = k_cache.reshape(nb * bs, hkv, d)
    fv = v_cache.reshape(nb * bs, hkv, d)
    slots = np.asarray(slot_mapping, dtype=np.int64)
    ok = (slots >= 0) & (slots < nb * bs)
    fk[slots[ok]] = np.asarray(k)[ok]
    fv[slots[ok]] = np.asarray(v)[ok]
    return k_cache, v_cache


# ----------------------------------------------------------------------------
# a6: block-table gather  (prefill...:79-82, decode...:69-71, qwen3.py:114-134)
# ----------------------------------------------------------------------------
def gather_kv(cache, block_tables, lengths):
    """Dense gather of each sequence's context through its block table.

    ``cache`` is the native per-layer pool ``[NB, BS, Hkv, d]``;
    ``ctx[b, j] = cache[bt[b, j // BS], j % BS]`` for ``j < lengths[b]``
    (``_build_slots`` qwen3.py:114-117 with the clip at :129-131); rows
    ``j >= lengths[b]`` are zero.  Negative table entries read block 0, like
    ``safe_block_tables`` (qwen3.py:179-180, prefill...:80).

    Returns ``[B, P*BS, Hkv, d]`` with the cache's dtype.
    """
    cache = np.asarray(cache)
    bt = np.asarray(block_tables, dtype=np.int64)
    nb, bs, hkv, d = cache.shape
    b, p = bt.shape
    safe = np.where(bt >= 0, bt, 0)
    out = cache[safe].reshape(b, p * bs, hkv, d).copy()
    j = np.arange(p * bs)[None, :]
    out[j >= np.asarray(lengths)[:, None]] = 0
    return out


# ----------------------------------------------------------------------------
# reference tiling helpers
# ----------------------------------------------------------------------------
def largest_divisor_at_most(value: int, upper: int) -> int:
    """prefill_paged_attention.py:153-157."""
    for cand in (16, 8, 4, 2, 1):
        if cand <= upper and value % cand == 0:
            return cand
    return 1


def decode_k_splits(pages_per_sequence: int) -> int:
    """The caller's split choice for decode (qwen3.py:201-206)."""
    for cand in (16, 8, 4, 2):
        if pages_per_sequence % cand == 0:
            return cand
    return 1


def _split_attention_rows(qs, k_ctx, v_ctx, valid, *, k_splits, block_k,
                          page_size, used_tokens, soft_cap, mask_value, k_scale=None, v_scale=None):
    """One q-row block against one kv head's context, reference algebra.

    Restates the kernel body shared by prefill (prefill...:62-150) and decode
    (decode...:57-149): the context is cut into ``k_splits`` partitions of
    ``pages_per_partition`` pages; each partition runs an online softmax over
    compute blocks of ``block_k`` tokens with exp2/log2e, P cast to bf16
    before PV, and writes partial ``o`` as bf16 with f32 ``l``, ``m``.
    Partitions that start past the used pages are skipped
    (prefill...:66-69,135-139; decode...:130-142).

    qs:    [R, d] f32 (already scaled, bf16-valued)
    k_ctx: [Pmax*BS, d] f32 context in block-table order
    valid: [R, Pmax*BS] bool mask (length, causal, row-in-range)
    k_scale / v_scale: optional [Pmax*BS] f32 per-token scales of quantized
    pages (decode...:72-81,108-115; prefill...:84-92,120-123): logits are
    multiplied by k_scale before the soft cap, and PV uses the float32
    ``P * v_scale`` against float32 V (no bf16 rounding of P).
    Returns (o_parts bf16-valued f32 [S,R,d], l [S,R], m [S,R]).
    """
    r, d = qs.shape
    total = k_ctx.shape[0]
    pages_total = total // page_size
    ppp = pages_total // k_splits
    used_pages = -(-used_tokens // page_size)
    o_parts = np.zeros((k_splits, r, d), np.float32)
    l_parts = np.zeros((k_splits, r), np.float32)
    m_parts = np.full((k_splits, r), F32_MIN, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        return _split_loop(qs, k_ctx, v_ctx, valid, o_parts, l_parts, m_parts, k_splits=k_splits,
                           ppp=ppp, used_pages=used_pages, block_k=block_k, page_size=page_size,
                           soft_cap=soft_cap, mask_value=mask_value, k_scale=k_scale, v_scale=v_scale)


def _split_loop(qs, k_ctx, v_ctx, valid, o_parts, l_parts, m_parts, *, k_splits, ppp, used_pages,
                block_k, page_size, soft_cap, mask_value, k_scale=None, v_scale=None):
    r, d = qs.shape
    total = k_ctx.shape[0]
    for s in range(k_splits):
        start_page = s * ppp
        end_page = min(start_page + ppp, used_pages)
        if start_page >= end_page:
            continue
        m_i = np.full(r, F32_MIN, np.float32)
        l_i = np.zeros(r, np.float32)
        o = np.zeros((r, d), np.float32)
        n_blocks = -(-(end_page - start_page) * page_size // block_k)
        for it in range(n_blocks):
            t0 = start_page * page_size + it * block_k
            t1 = t0 + block_k
            # Compute blocks may run past the partition (and past the table);
            # those tokens are masked by length (prefill...:103-107).
            kb = np.zeros((block_k, d), np.float32)
            vb = np.zeros((block_k, d), np.float32)
            hi = min(t1, total)
            kb[: hi - t0] = k_ctx[t0:hi]
            vb[: hi - t0] = v_ctx[t0:hi]
            logits = qs @ kb.T
            if k_scale is not None:
                ksb = np.zeros(block_k, np.float32)
                ksb[: hi - t0] = k_scale[t0:hi]
                logits = (logits * ksb[None, :]).astype(np.float32)
            if soft_cap is not None:
                logits = (np.tanh(logits / np.float32(soft_cap)) * np.float32(soft_cap)).astype(np.float32)
            mask = np.zeros((r, block_k), bool)
            mask[:, : hi - t0] = valid[:, t0:hi]
            logits = np.where(mask, logits, np.float32(mask_value)).astype(np.float32)
            m_curr = logits.max(axis=-1)
            m_next = np.maximum(m_i, m_curr)
            corr = np.exp2((m_i - m_next) * np.float32(LOG2E)).astype(np.float32)
            s_curr = np.exp2((logits - m_next[:, None]) * np.float32(LOG2E)).astype(np.float32)
            l_i = (corr * l_i + s_curr.sum(axis=-1, dtype=np.float32)).astype(np.float32)
            if v_scale is not None:
                vsb = np.zeros(block_k, np.float32)
                vsb[: hi - t0] = v_scale[t0:hi]
                o = corr[:, None] * o + (s_curr * vsb[None, :]).astype(np.float32) @ vb
            else:
                o = corr[:, None] * o + round_bf16(s_curr) @ vb
            m_i = m_next
        o_parts[s] = round_bf16(o)
        l_parts[s] = l_i
        m_parts[s] = m_i
    return o_parts, l_parts, m_parts


def _merge_splits(o_parts, l_parts, m_parts):
    """Final log-sum-exp merge across splits in the reference's dtypes.

    prefill...:371-376 and decode...:274-282: ``m* = max m_s``;
    ``o = sum_s bf16(o_s * bf16(e^{m_s - m*})) / bf16(sum_s l_s e^{m_s-m*} + eps)``.
    """
    m_next = m_parts.max(axis=0)
    corr = np.exp((m_parts - m_next[None]).astype(np.float64)).astype(np.float32)
    o = round_bf16(o_parts * round_bf16(corr)[..., None])
    l_next = (l_parts * corr).sum(axis=0, dtype=np.float32)
    num = round_bf16(o.sum(axis=0, dtype=np.float32))
    den = round_bf16(l_next + np.float32(F32_EPS))
    with np.errstate(invalid="ignore", divide="ignore"):
        out = round_bf16(num / den[..., None])
    return out


# ----------------------------------------------------------------------------
# a4: prefill  (prefill_paged_attention.py:18-150, 160-388)
# ----------------------------------------------------------------------------
def prefill_attention(q, k_pages, v_pages, block_tables, cu_seqlens,
                      input_positions, *, cu_seqlens_k=None, k_splits=8,
                      pages_per_compute_block=8, soft_cap=None,
                      mask_value=DEFAULT_MASK_VALUE, rows=None, k_scales_pages=None, v_scales_pages=None,
                      code_type="e4m3"):
    """Ragged causal GQA paged prefill, restating the reference kernel.

    Layouts follow the reference kernel entry (prefill...:407-429):
    q ``[T, H, d]``; k_pages / v_pages ``[Hkv, NB, BS, d]``; block_tables
    ``[B, P]`` int32 (negative entries read block 0, qwen3.py:179-180);
    cu_seqlens ``[B+1]``; input_positions ``[T]``.

    Semantics (prefill...:52-60,100-107,227-230,384-388):
      * sequence b owns q rows ``cu[b]:cu[b+1]``;
      * q is scaled in bf16: ``bf16(q * bf16(1/sqrt(d)))`` (prefill...:60);
      * kv index j of sequence b has position ``j + pos0_b`` with
        ``pos0_b = input_positions[cu[b]]`` and is visible to row i iff
        ``j < L_b`` and ``j + pos0_b <= input_positions[i]``;
      * GQA: q head h reads kv head ``h // G`` (prefill...:209-211);
      * rows outside every sequence are 0;
      * a row of a sequence that sees no kv index (its position precedes the
        sequence's first kv position) is 0, the value the reference's dense
        definition gives it (prefill...:502, qwen3.py:166).  The Pallas
        kernel differs there: its finite ``mask_value`` with ``m`` starting
        at ``f32.min`` (prefill...:62-64,109-117) weighs every token of the
        loaded compute blocks equally, a mean of V that includes tokens past
        the sequence.  The engine never builds such a row (positions run
        0, 1, 2, ... per sequence, model_runner.py:228).

    ``cu_seqlens_k`` (optional) extends the reference to a cached prefix: the
    kv length becomes ``Lk_b = cu_k[b+1]-cu_k[b]`` and kv index j has position
    ``j + pos0_b - (Lk_b - L_b)``.  With ``cu_seqlens_k == cu_seqlens`` this is
    exactly the reference rule.

    ``rows`` (optional int array) restricts the computation to those q rows
    (other rows of the result stay 0) so large workloads can be sampled.
    Quantized pages (prefill...:169-170,255-266, in-kernel :84-92,120-123):
    1-byte codes with ``[Hkv, NB, BS]`` float32 per-token scales, as in
    decode_attention (``code_type``).
    Returns bf16 bit patterns ``[T, H, d]``.
    """
    qf = _as_f32(q)
    quant = k_scales_pages is not None
    kp = np.asarray(k_pages)
    vp = np.asarray(v_pages)
    if quant:
        ksp = np.asarray(k_scales_pages, np.float32)
        vsp = np.asarray(v_scales_pages, np.float32)
    t_total, h, d = qf.shape
    hkv, nb, bs, _ = kp.shape
    g = h // hkv
    bt = np.asarray(block_tables, dtype=np.int64)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    cuk = cu if cu_seqlens_k is None else np.asarray(cu_seqlens_k, dtype=np.int64)
    pos = np.asarray(input_positions, dtype=np.int64)
    b_count, p = bt.shape
    ks = largest_divisor_at_most(p, k_splits)
    ppp = p // ks
    ppcb = largest_divisor_at_most(ppp, min(ppp, pages_per_compute_block))
    block_k = ppcb * bs
    # q * (1/sqrt(d)) under JAX weak typing: the scalar becomes bf16 first.
    scale = float(round_bf16(np.float32(1.0 / math.sqrt(d))).reshape(-1)[0])
    qs_all = round_bf16(qf * np.float32(scale))
    out = np.zeros((t_total, h, d), np.float32)
    row_sel = None if rows is None else np.zeros(t_total, bool)
    if rows is not None:
        row_sel[np.asarray(rows, dtype=np.int64)] = True
    safe = np.where(bt >= 0, bt, 0)
    for b in range(b_count):
        q0, q1 = int(cu[b]), int(cu[b + 1])
        lq = q1 - q0
        if lq <= 0:
            continue
        lk = int(cuk[b + 1] - cuk[b])
        if lk <= 0:
            continue
        sel = np.arange(q0, q1)
        if row_sel is not None:
            sel = sel[row_sel[q0:q1]]
            if sel.size == 0:
                continue
        pos0 = int(pos[q0]) - (lk - lq)
        kv_pos = np.arange(p * bs) + pos0
        q_pos = pos[sel]
        valid = (np.arange(p * bs)[None, :] < lk) & (kv_pos[None, :] <= q_pos[:, None])
        for kh in range(hkv):
            if quant:
                k_ctx = code_values(kp[kh][safe[b]].reshape(p * bs, d), code_type)
                v_ctx = code_values(vp[kh][safe[b]].reshape(p * bs, d), code_type)
                k_sc = ksp[kh][safe[b]].reshape(p * bs)
                v_sc = vsp[kh][safe[b]].reshape(p * bs)
            else:
                k_ctx = _as_f32(kp[kh][safe[b]].reshape(p * bs, d))
                v_ctx = _as_f32(vp[kh][safe[b]].reshape(p * bs, d))
                k_sc = v_sc = None
            qs = qs_all[sel, kh * g:(kh + 1) * g].reshape(-1, d)
            vmask = np.repeat(valid, g, axis=0)
            o_p, l_p, m_p = _split_attention_rows(
                qs, k_ctx, v_ctx, vmask, k_splits=ks, block_k=block_k,
                page_size=bs, used_tokens=lk, soft_cap=soft_cap,
                mask_value=mask_value, k_scale=k_sc, v_scale=v_sc)
            res = _merge_splits(o_p, l_p, m_p)
            res = np.where(vmask.any(axis=1)[:, None], res, np.float32(0))  # rows with no visible key
            out[sel, kh * g:(kh + 1) * g] = res.reshape(sel.size, g, d)
    return f32_to_bf16(out)


# ----------------------------------------------------------------------------
# a5: decode  (decode_paged_attention.py:34-149, 152-283, 300-397)
# ----------------------------------------------------------------------------
def decode_attention(q, k_pages, v_pages, block_tables, lengths, *,
                     k_splits=None, pages_per_compute_block=8, soft_cap=None,
                     mask_value=DEFAULT_MASK_VALUE, seqs=None, k_scales_pages=None, v_scales_pages=None,
                     code_type="e4m3"):
    """Split-K paged GQA decode, restating the reference kernel.

    q ``[B, H, d]`` is used as given -- the reference kernel applies no scale;
    its caller pre-scales q in bf16 (qwen3.py:207).  ``lengths[b]`` counts
    the visible context (kv index ``j < lengths[b]``, decode...:88-97);
    length 0 gives 0 (decode...:136-142 then 0/(0+eps)).  ``k_splits`` defaults
    to the caller's choice (qwen3.py:201-206); ``pages_per_compute_block`` is
    ``min(ppp, 8)`` and must divide the partition (decode...:179-184).

    ``seqs`` (optional) restricts the computation to those sequences.
    Quantized pages (decode...:158-159,206-217): ``k_pages`` / ``v_pages``
    hold 1-byte codes -- ``code_type`` "e4m3" (float8 e4m3fn bit patterns),
    "int8" or "uint8" (integers; the reference's ``astype`` to q's dtype
    keeps the integer value) -- and ``k_scales_pages`` / ``v_scales_pages``
    ``[Hkv, NB, BS]`` float32 per-token scales; K is cast to bf16 exactly
    (decode...:72-74), V to float32 (decode...:108-115).
    Returns bf16 bit patterns ``[B, H, d]``.
    """
    qf = round_bf16(_as_f32(q))
    quant = k_scales_pages is not None
    kp = np.asarray(k_pages)
    vp = np.asarray(v_pages)
    if quant:
        ksp = np.asarray(k_scales_pages, np.float32)
        vsp = np.asarray(v_scales_pages, np.float32)
    b_count, h, d = qf.shape
    hkv, nb, bs, _ = kp.shape
    g = h // hkv
    bt = np.asarray(block_tables, dtype=np.int64)
    p = bt.shape[1]
    lens = np.asarray(lengths, dtype=np.int64)
    ks = decode_k_splits(p) if k_splits is None else k_splits
    if p % ks:
        raise ValueError(f"pages_per_sequence={p} must be divisible by k_splits={ks}")
    ppp = p // ks
    ppcb = min(ppp, pages_per_compute_block)
    if ppp % ppcb:
        raise ValueError(f"pages_per_partition={ppp} must be divisible by {ppcb}")
    block_k = ppcb * bs
    safe = np.where(bt >= 0, bt, 0)
    out = np.zeros((b_count, h, d), np.float32)
    seq_iter = range(b_count) if seqs is None else [int(s) for s in seqs]
    for b in seq_iter:
        ln = int(lens[b])
        valid = np.arange(p * bs)[None, :] < ln
        for kh in range(hkv):
            if ln <= 0:
                continue
            if quant:
                k_ctx = code_values(kp[kh][safe[b]].reshape(p * bs, d), code_type)
                v_ctx = code_values(vp[kh][safe[b]].reshape(p * bs, d), code_type)
                k_sc = ksp[kh][safe[b]].reshape(p * bs)
                v_sc = vsp[kh][safe[b]].reshape(p * bs)
            else:
                k_ctx = _as_f32(kp[kh][safe[b]].reshape(p * bs, d))
                v_ctx = _as_f32(vp[kh][safe[b]].reshape(p * bs, d))
                k_sc = v_sc = None
            qs = qf[b, kh * g:(kh + 1) * g]
            vmask = np.repeat(valid, g, axis=0)
            o_p, l_p, m_p = _split_attention_rows(
                qs, k_ctx, v_ctx, vmask, k_splits=ks, block_k=block_k,
                page_size=bs, used_tokens=ln, soft_cap=soft_cap,
                mask_value=mask_value, k_scale=k_sc, v_scale=v_sc)
            out[b, kh * g:(kh + 1) * g] = _merge_splits(o_p, l_p, m_p)
    return f32_to_bf16(out)


# ----------------------------------------------------------------------------
# brute force (float64) -- the pin for the two functions above
# ----------------------------------------------------------------------------
def dense_prefill_f64(q, k_ctx, v_ctx, cu_seqlens, input_positions, *,
                      cu_seqlens_k=None, scale=None, soft_cap=None):
    """Dense masked softmax attention in float64 on tiny inputs.

    Mask definition of ``prefill_paged_attention_reference``
    (prefill...:487-492) applied per sequence: same sequence, kv position
    <= q position.  ``k_ctx``/``v_ctx`` are per-sequence dense contexts
    ``[B, Lk_max, Hkv, d]`` (e.g. from :func:`gather_kv`).  Fully masked rows
    and rows outside every sequence are 0 (prefill...:502, qwen3.py:166).
    """
    qf = _as_f32(q).astype(np.float64)
    kf = _as_f32(k_ctx).astype(np.float64)
    vf = _as_f32(v_ctx).astype(np.float64)
    t_total, h, d = qf.shape
    hkv = kf.shape[2]
    g = h // hkv
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    cuk = cu if cu_seqlens_k is None else np.asarray(cu_seqlens_k, dtype=np.int64)
    pos = np.asarray(input_positions, dtype=np.int64)
    sc = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((t_total, h, d), np.float64)
    for b in range(len(cu) - 1):
        q0, q1 = int(cu[b]), int(cu[b + 1])
        lq, lk = q1 - q0, int(cuk[b + 1] - cuk[b])
        if lq <= 0 or lk <= 0:
            continue
        kv_pos = np.arange(lk) + int(pos[q0]) - (lk - lq)
        for i in range(q0, q1):
            vis = kv_pos <= pos[i]
            if not vis.any():
                continue
            for hh in range(h):
                kh = hh // g
                s = kf[b, :lk, kh] @ qf[i, hh] * sc
                if soft_cap is not None:
                    s = np.tanh(s / soft_cap) * soft_cap
                s = np.where(vis, s, -np.inf)
                w = np.exp(s - s.max())
                w /= w.sum()
                out[i, hh] = w @ vf[b, :lk, kh]
    return out


def dense_decode_f64(q, k_ctx, v_ctx, lengths, *, scale=1.0, soft_cap=None):
    """Dense decode attention in float64 (``paged_attention_reference``,
    decode...:426-463): mask ``j < lengths[b]``; length 0 gives 0."""
    qf = _as_f32(q).astype(np.float64)
    kf = _as_f32(k_ctx).astype(np.float64)
    vf = _as_f32(v_ctx).astype(np.float64)
    b_count, h, d = qf.shape
    hkv = kf.shape[2]
    g = h // hkv
    out = np.zeros((b_count, h, d), np.float64)
    for b in range(b_count):
        ln = int(lengths[b])
        if ln <= 0:
            continue
        for hh in range(h):
            kh = hh // g
            s = kf[b, :ln, kh] @ qf[b, hh] * scale
            if soft_cap is not None:
                s = np.tanh(s / soft_cap) * soft_cap
            w = np.exp(s - s.max())
            w /= w.sum()
            out[b, hh] = w @ vf[b, :ln, kh]
    return out


# ----------------------------------------------------------------------------
# algorithmic work (roofline accounting)
# ----------------------------------------------------------------------------
def prefill_visible_pairs(cu_seqlens, cu_seqlens_k=None) -> int:
    """sum_b N_b*P_b + N_b(N_b+1)/2 for positions restarting per sequence."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    cuk = cu if cu_seqlens_k is None else np.asarray(cu_seqlens_k, dtype=np.int64)
    n = np.diff(cu)
    pfx = np.diff(cuk) - n
    return int((n * pfx + n * (n + 1) // 2).sum())


# ----------------------------------------------------------------------------
# f1: QK RMSNorm + RoPE + KV store, the layer step before attention
#     (qwen3.py:286-299 with apply_rope qwen3.py:59-78)
# ----------------------------------------------------------------------------
def rope_inv_freq(head_dim: int, rope_theta: float) -> np.ndarray:
    """``1 / rope_theta ** (arange(0, d, 2, bf16) / d)`` as the reference
    evaluates it (qwen3.py:62-63): every operand and result is bf16, so the
    weakly typed ``rope_theta`` is rounded to bf16 first (1e6 -> 999424) and
    each of arange/d, the power and the reciprocal is rounded to bf16.
    Returns float32 values (all representable in bf16), shape [d/2]."""
    e = round_bf16(np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim))
    theta = round_bf16(np.float32(rope_theta)).reshape(-1)[0]
    p = round_bf16(np.power(theta, e, dtype=np.float32))
    return round_bf16(np.float32(1.0) / p)


def rope_positions(positions, rope_scaling=None) -> np.ndarray:
    """``_maybe_scale_positions`` then ``.astype(bf16)`` (qwen3.py:48-56,61):
    linear/dynamic scaling divides by the factor in float32, then positions
    are rounded to bf16 (exact only up to 256)."""
    pos = np.asarray(positions).astype(np.float32)
    if rope_scaling is not None and rope_scaling.get("type") in {"linear", "dynamic"}:
        pos = pos / np.float32(rope_scaling.get("factor", 1.0))
    return round_bf16(pos)


def rope_cos_sin(positions, head_dim: int, rope_theta: float, rope_scaling=None):
    """cos/sin tables [T, d/2] (qwen3.py:64-66): freqs = bf16(pos x inv_freq),
    cos/sin evaluated in float32 and rounded to bf16."""
    pos = rope_positions(positions, rope_scaling)
    inv = rope_inv_freq(head_dim, rope_theta)
    freqs = round_bf16(pos[:, None] * inv[None, :])
    return round_bf16(np.cos(freqs)), round_bf16(np.sin(freqs))


def apply_rope(x, cos, sin) -> np.ndarray:
    """Rotate interleaved pairs (x[2i], x[2i+1]) (qwen3.py:68-73):
    (x1 cos - x2 sin, x1 sin + x2 cos), written back interleaved.  x: bf16
    bits [T, heads, d]; cos/sin: [T, d/2].  The rotation is evaluated in
    float32 and rounded once to bf16."""
    xf = _as_f32(x)
    x1, x2 = xf[..., 0::2], xf[..., 1::2]
    c, s = cos[:, None, :], sin[:, None, :]
    out = np.empty_like(xf)
    out[..., 0::2] = x1 * c - x2 * s
    out[..., 1::2] = x1 * s + x2 * c
    return f32_to_bf16(out)


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """flax ``nnx.RMSNorm`` over the last axis as the reference layer uses it
    (qwen3.py:235-241,287,293): mean of squares in float32,
    ``y = x * (rsqrt(mean + eps) * weight)`` in float32, rounded to bf16."""
    xf = _as_f32(x)
    w = _as_f32(weight)
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=np.float32)
    mul = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32) * w
    return f32_to_bf16(xf * mul)


def qk_norm_rope_store(q, k, v, q_norm_w, k_norm_w, positions, slot_mapping, k_cache, v_cache, *,
                       eps: float, rope_theta: float, rope_scaling=None):
    """The layer step before attention (qwen3.py:286-299): q and k get RMSNorm
    then RoPE; k and v are stored into the pool through the slot mapping
    (``_update_kv_cache``, qwen3.py:105-111).  Returns (q_out, k_cache,
    v_cache); bf16 bit patterns throughout."""
    d = np.asarray(q).shape[-1]
    cos, sin = rope_cos_sin(positions, d, rope_theta, rope_scaling)
    q_out = apply_rope(rms_norm(q, q_norm_w, eps), cos, sin)
    k_out = apply_rope(rms_norm(k, k_norm_w, eps), cos, sin)
    kc, vc = kv_store(k_cache, v_cache, k_out, v, slot_mapping)
    return q_out, kc, vc


# ----------------------------------------------------------------------------
# f2: one scheduler step with decode and prefill sequences
#     (model_runner.py:310-333 runs them as two calls: decode, then prefill)
# ----------------------------------------------------------------------------
def mixed_attention(q, k_pages, v_pages, block_tables, cu_seqlens_q, kv_lens, input_positions,
                    num_decodes: int, *, soft_cap=None, prefill_rows=None, decode_seqs=None):
    """The reference step's two attention calls over one unpadded batch.

    Sequences ``b < num_decodes`` are decode sequences: their q row
    ``cu_seqlens_q[b]`` is scaled as the decode caller does it,
    ``bf16(q / bf16(sqrt(d)))`` (qwen3.py:207), and attends to kv indices
    ``j < kv_lens[b]`` (decode_attention above).  The others are prefill
    sequences with kv length ``kv_lens[b]`` (prefill_attention above with
    ``cu_seqlens_k`` built from kv_lens).  Rows no sequence computes are 0.
    ``prefill_rows`` (rows of q, optional) and ``decode_seqs`` (optional)
    restrict the work for sampling.  Returns bf16 bit patterns ``[T, H, d]``.
    """
    qf = _as_f32(q)
    t_total, h, d = qf.shape
    bt = np.asarray(block_tables)
    cu = np.asarray(cu_seqlens_q, dtype=np.int64)
    kl = np.asarray(kv_lens, dtype=np.int64)
    pos = np.asarray(input_positions)
    nd = int(num_decodes)
    out = np.zeros((t_total, h, d), np.uint16)
    if nd > 0:
        root = float(round_bf16(np.float32(math.sqrt(d))).reshape(-1)[0])
        dec_rows = cu[:nd]
        has_row = (cu[1:nd + 1] > cu[:nd]) & (cu[:nd] < t_total)
        seqs = np.nonzero(has_row)[0]
        if decode_seqs is not None:
            seqs = np.intersect1d(seqs, np.asarray(decode_seqs))
        qd = np.zeros((nd, h, d), np.float32)
        qd[seqs] = qf[dec_rows[seqs]]
        qd = round_bf16(qd / np.float32(root))
        od = decode_attention(qd, k_pages, v_pages, bt[:nd], kl[:nd], soft_cap=soft_cap, seqs=seqs)
        out[dec_rows[seqs]] = od[seqs]
    if nd < len(kl):
        base = int(cu[nd])
        cu_p = cu[nd:] - base
        cuk = np.concatenate([[0], np.cumsum(kl[nd:])])
        rows = None
        if prefill_rows is not None:
            rows = np.asarray(prefill_rows, dtype=np.int64) - base
        tail = prefill_attention(qf[base:], k_pages, v_pages, bt[nd:], cu_p, pos[base:], cu_seqlens_k=cuk,
                                 soft_cap=soft_cap, rows=rows)
        sel = slice(base, base + int(cu_p[-1]))
        out[sel] = tail[:int(cu_p[-1])]
    return out


# ----------------------------------------------------------------------------
# f4: float8 e4m3fn KV pages with per-token scales
# ----------------------------------------------------------------------------
def _e4m3_table() -> np.ndarray:
    """Values of the 256 OCP float8 e4m3fn codes (1 sign, 4 exponent bits with
    bias 7, 3 mantissa bits; no infinities; 0x7f / 0xff are NaN)."""
    c = np.arange(256)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    v = sign * mag
    v[(c & 0x7F) == 0x7F] = np.nan
    return v.astype(np.float32)


_E4M3 = _e4m3_table()
E4M3_MAX = 448.0


def fp8_e4m3_decode(codes) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values (exact)."""
    return _E4M3[np.asarray(codes, dtype=np.uint8)]


def code_values(codes, code_type="e4m3") -> np.ndarray:
    """Values of 1-byte page codes as the reference's cast sees them
    (decode...:72-75,108-115; prefill...:84-85,118-123): "e4m3" float8
    e4m3fn bit patterns, "int8" / "uint8" the integers (codes may be given
    as int8 or as their uint8 bit patterns); exact in float32 and bf16."""
    c = np.asarray(codes)
    if code_type == "e4m3":
        return fp8_e4m3_decode(c.view(np.uint8) if c.dtype == np.int8 else c)
    if code_type == "int8":
        return (c if c.dtype == np.int8 else c.astype(np.uint8).view(np.int8)).astype(np.float32)
    if code_type == "uint8":
        return (c.view(np.uint8) if c.dtype == np.int8 else c.astype(np.uint8)).astype(np.float32)
    raise ValueError(f"unknown code_type {code_type!r}")


def fp8_e4m3_encode(x) -> np.ndarray:
    """float32 -> e4m3fn codes, round to nearest, ties to the even code,
    negative values keeping the sign bit (so -0 for a negative underflow);
    magnitudes above 448 saturate to 448 (the quantizer below never
    produces them)."""
    x = np.asarray(x, dtype=np.float32)
    pos = _E4M3[:0x7F].astype(np.float64)          # codes 0..126, increasing
    a = np.minimum(np.abs(x).astype(np.float64), E4M3_MAX)
    hi = np.clip(np.searchsorted(pos, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo, dhi = a - pos[lo], pos[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)   # -0 stays -0


def quantize_fp8_rows(x):
    """Per-row float8 quantisation of bf16 rows ``[..., d]`` (bit patterns):
    ``amax = max |x|``; the stored scale is the smallest power of two
    ``s = 2^e`` with ``amax / s <= 448``, but at least ``2^-126`` (a normal
    float); the codes are ``e4m3(x / s)`` (the division by a power of two is
    exact).  An all-zero row stores scale 1 and zero codes.  Returns (codes
    uint8 [..., d], scales float32 [...]).  This is the library's own
    quantiser (the reference reads quantized pages but has no writer); a
    power-of-two scale lets a reader widen code and scale in one exact step."""
    xf = _as_f32(x)
    amax = np.abs(xf).max(axis=-1).astype(np.float64)
    nz = amax > 0
    # smallest e with amax <= 448 * 2^e, found from an estimate by exact
    # float64 comparisons (448 * 2^e is exact)
    est = np.where(nz, np.ceil(np.log2(np.where(nz, amax, 1.0) / E4M3_MAX)), 0.0).astype(np.int64)
    e = est.copy()
    for _ in range(3):
        e = np.where(nz & (amax > E4M3_MAX * np.exp2(e.astype(np.float64))), e + 1, e)
    for _ in range(3):
        e = np.where(nz & (amax <= E4M3_MAX * np.exp2((e - 1).astype(np.float64))), e - 1, e)
    e = np.maximum(e, -126)
    scale = np.where(nz, np.exp2(e.astype(np.float64)), 1.0).astype(np.float32)
    inv = np.where(nz, np.exp2(-e.astype(np.float64)), 1.0).astype(np.float32)
    codes = fp8_e4m3_encode((xf * inv[..., None]).astype(np.float32))
    return codes, scale


def kv_store_fp8(k_codes, v_codes, k_scales, v_scales, k, v, slot_mapping):
    """Quantised KV store: the rows of token t go to flat slot
    ``slot_mapping[t]`` (skipped outside the pool, as kv_store above).
    Pools: codes ``[NB, BS, Hkv, d]`` uint8, scales ``[Hkv, NB, BS]`` float32
    (the layout of k_scales_pages, decode...:206-217)."""
    kc, vc = np.array(k_codes, copy=True), np.array(v_codes, copy=True)
    ks, vs = np.array(k_scales, copy=True), np.array(v_scales, copy=True)
    nb, bs, hkv, d = kc.shape
    kq, kscale = quantize_fp8_rows(k)
    vq, vscale = quantize_fp8_rows(v)
    for t, slot in enumerate(np.asarray(slot_mapping, dtype=np.int64)):
        if slot < 0 or slot >= nb * bs:
            continue
        pg, off = divmod(int(slot), bs)
        kc[pg, off], vc[pg, off] = kq[t], vq[t]
        ks[:, pg, off], vs[:, pg, off] = kscale[t], vscale[t]
    return kc, vc, ks, vs
