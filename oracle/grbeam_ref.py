"""CPU restatement of GRBeam fixed-depth beam search (oracle; tests only).

Follows src/kadllm/grbeam.py:45-105.  ``grbeam_search`` drives any object
with ``prefill(ids) -> (logits[B,V], state)`` and ``decode(history, state)
-> logits[B,W,V]``.  Selection is per request: full-vocabulary fp32
log-softmax, optional bool mask (True = allowed, no renormalisation), add the
parent score, flatten [W*V] and take the top ``width`` (sorted descending).

Ties: torch.topk leaves tie order unspecified (grbeam.py:95).  This oracle
breaks ties by the lower flat index, the rule the HIP selection kernel
implements, so that tie-free inputs compare exactly and tied inputs compare
deterministically.
"""

import itertools

import torch


def select_topk(flat_scores, width):
    """Top ``width`` of a 1-D fp32 tensor, descending, ties to the lower index."""
    n = flat_scores.numel()
    order = sorted(range(n), key=lambda i: (-float(flat_scores[i]), i)) if n <= 4096 else None
    if order is None:
        # stable sort on (-score) keeps index order among equal scores
        idx = torch.sort(-flat_scores, stable=True).indices[:width]
        return flat_scores[idx], idx
    idx = torch.tensor(order[:width], dtype=torch.int64)
    return flat_scores[idx], idx


def level_select(logits, scores, width, mask=None):
    """One GRBeam level for all requests (src/kadllm/grbeam.py:89-104).

    logits [B,Wp,V] (any float dtype), scores [B,Wp] fp32, mask [B,Wp,V] bool
    or None.  Returns (new_scores [B,width], parents [B,width], tokens [B,width]).
    """
    B, Wp, V = logits.shape
    out_s, out_i = [], []
    for r in range(B):
        logp = logits[r].float().log_softmax(-1)
        if mask is not None:
            logp = logp.masked_fill(~mask[r], -torch.inf)
        logp = logp + scores[r, :, None]
        s, i = select_topk(logp.reshape(-1), width)
        out_s.append(s)
        out_i.append(i)
    s = torch.stack(out_s)
    i = torch.stack(out_i)
    return s, i // V, i % V


def grbeam_search(adapter, input_ids, widths, *, allowed=None):
    """Fixed-depth GRBeam search (src/kadllm/grbeam.py:45-105).

    Returns (tokens [B,W_last,depth] int64, scores [B,W_last] fp32,
    valid [B,W_last] bool, per_level_logits list).
    """
    logits0, state = adapter.prefill(input_ids)
    B = input_ids.shape[0]
    V = logits0.shape[-1]
    history = input_ids.new_empty(B, 1, 0)
    scores = torch.zeros(B, 1)
    logits = logits0[:, None, :]
    seen = []
    for step, width in enumerate(widths):
        if step:
            logits = adapter.decode(history, state)
        seen.append(logits)
        mask = None if allowed is None else allowed(history, logits)
        if width > history.shape[1] * V:
            raise ValueError("beam width exceeds the number of candidate slots")
        scores, parents, tokens = level_select(logits, scores, width, mask)
        old = history.gather(1, parents[..., None].expand(B, width, step))
        history = torch.cat((old, tokens[..., None]), dim=-1)
    return history, scores, torch.isfinite(scores), seen


def brute_force_beam(logprob_fn, B, V, widths):
    """Exhaustive fixed-depth beam search for tiny vocabularies.

    ``logprob_fn(request, prefix_tuple) -> fp64 log-probs [V]`` of the next
    token.  Enumerates every sequence up to each depth, keeping at each level
    only the best ``widths[level]`` by cumulative log-prob (the definition of
    beam search), ties to the lexicographically lower (parent rank, token).
    Returns a list per request of (sequence tuple, cumulative score) lists.
    """
    results = []
    for r in range(B):
        beams = [((), 0.0)]
        for width in widths:
            cand = []
            for rank, (seq, sc) in enumerate(beams):
                lp = logprob_fn(r, seq)
                for tok in range(V):
                    cand.append((sc + float(lp[tok]), rank * V + tok, seq + (tok,)))
            cand.sort(key=lambda c: (-c[0], c[1]))
            beams = [(c[2], c[0]) for c in cand[:width]]
        results.append(beams)
    return results


def all_sequences(V, depth):
    return list(itertools.product(range(V), repeat=depth))


def level_select_grouped(logits, scores, groups, width, mask=None):
    """Per-group selection: each request's Wp rows form ``groups`` contiguous
    groups; every group keeps its ``width`` best candidates by cumulative
    full-vocabulary log-prob (ties to the lower (row, token) in the group).
    Returns (scores, parents, tokens) [B, groups * width], parents indexing the
    request's rows."""
    B, Wp, V = logits.shape
    rpg = Wp // groups
    s, p, t = level_select(logits.reshape(B * groups, rpg, V), scores.reshape(B * groups, rpg),
                           width, None if mask is None else mask.reshape(B * groups, rpg, V))
    p = p.view(B, groups, width) + torch.arange(groups)[:, None] * rpg
    return s.reshape(B, -1), p.reshape(B, -1), t.reshape(B, -1)


def conditional_search(adapter, input_ids, coarse_widths, fine_widths, *, allowed=None):
    """Two-level conditional search: ordinary levels over the full vocabulary
    (src/kadllm/grbeam.py:89-104), then levels in which every coarse beam keeps
    its own best ``fine_widths[i]`` descendants.  Returns (tokens, scores,
    valid, per-level logits)."""
    logits0, state = adapter.prefill(input_ids)
    B = input_ids.shape[0]
    V = logits0.shape[-1]
    history = input_ids.new_empty(B, 1, 0)
    scores = torch.zeros(B, 1)
    logits = logits0[:, None, :]
    seen = []
    groups = None
    levels = [(w, False) for w in coarse_widths] + [(w, True) for w in fine_widths]
    for step, (width, fine) in enumerate(levels):
        if step:
            logits = adapter.decode(history, state)
        seen.append(logits)
        mask = None if allowed is None else allowed(history, logits).expand(logits.shape)
        if fine:
            groups = history.shape[1] if groups is None else groups
            scores, parents, tokens = level_select_grouped(logits, scores, groups, width, mask)
        else:
            scores, parents, tokens = level_select(logits, scores, width, mask)
        old = history.gather(1, parents[..., None].expand(B, parents.shape[1], step))
        history = torch.cat((old, tokens[..., None]), dim=-1)
    return history, scores, torch.isfinite(scores), seen


def brute_force_conditional(logprob_fn, B, V, coarse_widths, fine_widths, allowed_fn=None):
    """Exhaustive conditional search for tiny vocabularies: the coarse levels
    are beam search by definition (best ``width`` cumulative log-probs over all
    expansions), then each coarse beam's subtree is searched on its own with
    the fine widths.  ``allowed_fn(request, prefix_tuple) -> bool [V]``;
    disallowed candidates score -inf and rank after every allowed one, ties to
    the lower (parent rank, token).  Returns per request a list of
    (sequence, score)."""
    def expand(r, beams, width):
        cand = []
        for rank, (seq, sc) in enumerate(beams):
            lp = logprob_fn(r, seq)
            ok = allowed_fn(r, seq) if allowed_fn is not None else None
            for tok in range(V):
                val = sc + float(lp[tok]) if ok is None or bool(ok[tok]) else float("-inf")
                cand.append((val, rank * V + tok, seq + (tok,)))
        cand.sort(key=lambda c: (-c[0], c[1]))
        return [(c[2], c[0]) for c in cand[:width]]

    results = []
    for r in range(B):
        beams = [((), 0.0)]
        for width in coarse_widths:
            beams = expand(r, beams, width)
        final = []
        for beam in beams:
            sub = [beam]
            for width in fine_widths:
                sub = expand(r, sub, width)
            final.extend(sub)
        results.append(final)
    return results
