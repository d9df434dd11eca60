"""A decoder init whose greedy tokens are decided by attention with a wide
margin (TEST INFRASTRUCTURE ONLY).

Two correct bf16 implementations of the same model differ in their logits
by rounding noise, so their greedy tokens can only be required to be
identical where the reference's top-2 logit gap is well above that noise.
With plain random weights the gap has no such floor (a fraction of a
percent of positions are near-ties). This init gives every position past
``offset`` a gap of several logit units while the token is still chosen by
the attention operator:

* every embedding row is a random direction of norm ``rho`` orthogonal to a
  fixed unit vector ``u``, plus ``beta * u``, so RMSNorm(embedding) has the
  same component along ``u`` for every token; the LM head is the embedding
  (tied, as in Qwen3; set equal for an untied model);
* layer 0's attention is a copy head: every query and key projection reads
  only the ``u`` component, so (after the optional q/k RMSNorm) queries and
  keys are the same vectors q0, k0 at every position and the rotary
  embedding alone sets the scores. q0/k0 place equal phase at a relative
  offset of ``offset`` on the 12 fastest rotary frequencies, weighted by
  sqrt(frequency): the score at that offset exceeds every other offset's (up
  to 40,000) by at least 16% of its value, and the value is set to ~160 (in
  softmax units), so the attention weight is 1 at position t - offset and
  below e^-25 anywhere else — the output there is that position's value row
  exactly, in any correct implementation;
* values and the output projection form a scaled orthogonal map, so the
  copy head adds ``gain`` times the normalised embedding of the token at
  t - offset to the residual stream;
* every other weight keeps the model's random init.

The greedy token at position t >= offset is then the token at position
t - offset: a wrong block, slot, position or mask in the attention path
changes the token, and the reference's top-2 gap at those positions is
several logit units (the tests assert the floor and report it).
"""

from __future__ import annotations

import math

import torch


def rotary_pattern(theta: float, head_dim: int, offset: int, pairs: int = 12) -> tuple[torch.Tensor, torch.Tensor]:
    """Unit-RMS q0, k0 (float64, [head_dim]) whose rotary scores peak at a
    query-minus-key distance of ``offset``; rotate-half pairs (i, i + D/2)."""

    half = head_dim // 2
    inv_freq = theta ** (-torch.arange(0, half, dtype=torch.float64) * 2 / head_dim)
    amp = inv_freq[:pairs].sqrt()
    q0 = torch.zeros(head_dim, dtype=torch.float64)
    k0 = torch.zeros(head_dim, dtype=torch.float64)
    angle = inv_freq[:pairs] * offset
    # score(d) = sum_i amp_i^2 cos(theta_i (d - offset)): the key rotates by
    # theta_i * s, the query by theta_i * t; the query's phase -theta_i * offset
    # aligns them at t - s = offset.
    k0[:pairs] = amp
    q0[:pairs] = amp * torch.cos(angle)
    q0[half : half + pairs] = -amp * torch.sin(angle)
    scale = math.sqrt(head_dim / (amp.square().sum().item()))
    return q0 * scale, k0 * scale


@torch.no_grad()
def make_copy_model(model, *, offset: int = 37, gain: float | None = None, peak_score: float = 160.0, seed: int = 1234):
    """Rewrite ``model``'s weights in place (see the module docstring).
    ``gain`` defaults to 4 * hidden / (KV heads * head_dim): the values span
    that fraction of the hidden space, so the copied embedding keeps the same
    share of its norm-squared margin."""

    c = model.config
    d, D = c.hidden_size, c.head_dim
    hq, hkv = c.num_attention_heads, c.num_key_value_heads
    if gain is None:
        gain = 4.0 * d / (hkv * D)
    group = hq // hkv
    dev, dt = model.device, model.dtype
    gen = torch.Generator(device="cpu").manual_seed(seed)

    u = (torch.randint(0, 2, (d,), generator=gen) * 2 - 1).to(torch.float64) / math.sqrt(d)
    rho = 0.02 * math.sqrt(d)
    beta = rho
    # Embedding rows: random directions orthogonal to u, norm rho, plus beta u.
    embed = torch.empty(c.vocab_size, d, dtype=dt, device=dev)
    for start in range(0, c.vocab_size, 16384):
        rows = torch.randn(min(16384, c.vocab_size - start), d, generator=gen, dtype=torch.float64)
        rows -= (rows @ u)[:, None] * u[None, :]
        rows *= rho / rows.norm(dim=1, keepdim=True)
        rows += beta * u[None, :]
        embed[start : start + rows.shape[0]] = rows.to(dt).to(dev)
    model.embed = embed
    model.lm_head = embed

    layer = model.layers[0]
    q0, k0 = rotary_pattern(c.rope_theta, D, offset)
    # Softmax units: q.k / sqrt(D); unit-RMS q0, k0 aligned give D / sqrt(D).
    if c.qk_norm:
        # The per-head RMSNorm removes the scalar u.x; its weight sets the scale.
        w = math.sqrt(peak_score / math.sqrt(D))
        qn, kn = q0, k0
        layer["q_norm"] = torch.full((D,), w, dtype=dt, device=dev)
        layer["k_norm"] = torch.full((D,), w, dtype=dt, device=dev)
    else:
        # u.x = beta sqrt(d) / sqrt(rho^2 + beta^2) for every token of layer 0.
        ux = beta * math.sqrt(d) / math.sqrt(rho * rho + beta * beta)
        a = math.sqrt(peak_score / math.sqrt(D)) / ux
        qn, kn = q0 * a, k0 * a
    q_rows = (qn[:, None] * u[None, :]).repeat(hq, 1)
    k_rows = (kn[:, None] * u[None, :]).repeat(hkv, 1)
    # Orthonormal rows for the values (hkv * D of them, hkv * D <= d).
    basis, _ = torch.linalg.qr(torch.randn(d, hkv * D, generator=gen, dtype=torch.float64))
    v_rows = basis.T  # [hkv * D, d]
    layer["qkv"] = torch.cat((q_rows, k_rows, v_rows)).to(dt).to(dev)
    # Output projection: query head j (KV head j // group) maps back through
    # its KV head's basis; the group's heads share the gain.
    o = torch.empty(d, hq * D, dtype=torch.float64)
    for j in range(hq):
        h = j // group
        o[:, j * D : (j + 1) * D] = basis[:, h * D : (h + 1) * D] * (gain / group)
    layer["o"] = o.to(dt).to(dev)
    return model
