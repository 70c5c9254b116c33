"""Bank maintenance of the reference's CPU/PyTorch path, restated.

TEST INFRASTRUCTURE ONLY (parity checker). Follows the non-Triton branches of
src/coda_gqa_l/memory_banks.py; the Triton branches (:617-632, :808-850) are
GPU-only and differ in semantics, so they are not restated.

All functions take the layer ``m`` (an OracleLayer: thresholds, sizes,
parameters) and the mutable state ``st`` and mutate ``st`` in place exactly
like the reference mixin does.  With a ``trace`` list they append their slot
decisions (the fields the golden vectors hold), followed by the masked
routing scores the decision was taken from (for margins in the tests).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .prims import unit

NEG_BIG = -(2 ** 62)


# --------------------------------------------------------------------------
# ring helpers
# --------------------------------------------------------------------------

def ring_time_order(m, st):
    """Recent ring in chronological order, memory_banks.py:135-150."""
    W = m.window
    n = int(st.recent_filled)
    kr, vr, gr = st.k_buf[:, :, :W], st.v_buf[:, :, :W], st.g_recent
    if n == 0:
        return kr[:, :, :0], vr[:, :, :0], gr[:, :0]
    if n < W:
        return kr[:, :, :n], vr[:, :, :n], gr[:, :n]
    i = int(st.recent_idx)
    return (torch.cat([kr[:, :, i:], kr[:, :, :i]], dim=2),
            torch.cat([vr[:, :, i:], vr[:, :, :i]], dim=2),
            torch.cat([gr[:, i:], gr[:, :i]], dim=1))


def ring_rebuild(m, st, k_seq, v_seq, g_seq):
    """Write a time-ordered ring at slots [0, Lr), zero the rest, memory_banks.py:152-177."""
    W = m.window
    Lr = k_seq.shape[2]
    if Lr > W:
        raise ValueError("k_seq longer than window")
    st.k_buf[:, :, :W].zero_()
    st.v_buf[:, :, :W].zero_()
    st.g_recent.zero_()
    st.allowed[:, :W].fill_(False)
    if Lr > 0:
        st.k_buf[:, :, :Lr] = k_seq
        st.v_buf[:, :, :Lr] = v_seq
        st.g_recent[:, :Lr] = g_seq.to(torch.float32)
        st.allowed[:, :Lr] = True
    st.recent_filled = int(Lr)
    st.recent_idx = 0


# --------------------------------------------------------------------------
# decode: one token
# --------------------------------------------------------------------------

def write_one(m, st, k_new, v_new, g_new, trace=None):
    """Ring write / evict for one token, memory_banks.py:183-224."""
    B = k_new.shape[0]
    W = m.window
    if st.recent_filled < W:
        j = int(st.recent_filled)
        st.k_buf[:, :, j:j + 1] = k_new
        st.v_buf[:, :, j:j + 1] = v_new
        st.g_recent[:, j:j + 1] = g_new
        st.allowed[:, j:j + 1] = True
        st.recent_filled += 1
    else:
        j = int(st.recent_idx)
        k_e = st.k_buf[:, :, j].detach()
        v_e = st.v_buf[:, :, j].detach()
        g_e = st.g_recent[:, j].detach()
        if st.metrics is not None:
            st.metrics["total_evictions"] += 1
        pos_e = torch.full((B,), int(st.pos - W), dtype=torch.int64)
        exact_one(m, st, k_e, v_e, pos_e, g_e, trace)
        summary_one(m, st, k_e, v_e, pos_e, g_e, trace)
        st.k_buf[:, :, j:j + 1] = k_new
        st.v_buf[:, :, j:j + 1] = v_new
        st.g_recent[:, j:j + 1] = g_new
        st.recent_idx = (j + 1) % W
    st.pos += 1


def exact_one(m, st, k_e, v_e, pos_e, gate, trace=None):
    """Exact bank, one evicted token, memory_banks.py:230-337."""
    if m.Me == 0:
        return
    B = k_e.shape[0]
    Me, Ae, W = m.Me, st.active_exact, m.window
    keep = gate >= m.write_gate_threshold_exact if m.write_policy != "none" else torch.ones(B, dtype=torch.bool)
    mem_k = st.k_buf[:, :, W:W + Me]
    mem_v = st.v_buf[:, :, W:W + Me]
    used = st.allowed[:, W:W + Me]

    sc = torch.einsum("bhd,bhmd->bhm", unit(v_e), st._exact_v_norm).mean(dim=1)
    if Ae < Me:
        sc[:, Ae:] = -1e9
    sc = sc.masked_fill(~used, -1e9)
    best, best_idx = sc.max(dim=-1)

    any_used = used[:, :Ae].any(dim=-1)
    novel = (~any_used) | (best < m.exact_novelty_threshold)
    hit = any_used & (best >= m.exact_match_threshold)

    free = ~used.clone()
    if Ae < Me:
        free[:, Ae:] = False
    free_exists = free.any(dim=-1)
    free_idx = free.to(torch.int64).argmax(dim=-1)
    last = st.mem_last_exact
    lm = torch.where(used, last, torch.full_like(last, 2 ** 62))
    if Ae < Me:
        lm[:, Ae:] = 2 ** 62
    lru_idx = lm.argmin(dim=-1)
    idx = torch.where(novel, torch.where(free_exists, free_idx, lru_idx), best_idx)

    ow = (novel | hit) if m.exact_refresh_on_hit else novel
    ow = ow & keep

    w = torch.zeros((B, Me), dtype=mem_k.dtype)
    w.scatter_(1, idx.view(B, 1), ow.to(mem_k.dtype).view(B, 1))
    w4 = w[:, None, :, None]
    new_k = mem_k + w4 * (k_e.unsqueeze(2) - mem_k)
    new_v = mem_v + w4 * (v_e.unsqueeze(2) - mem_v)
    new_used = used | w.to(torch.bool)
    st.k_buf[:, :, W:W + Me] = new_k
    st.v_buf[:, :, W:W + Me] = new_v
    st.allowed[:, W:W + Me] = new_used
    st._exact_v_norm = unit(new_v)

    if st.metrics is not None:
        mt = st.metrics
        if m.write_policy != "none":
            mt["tokens_gated_out"] += int((~keep).sum().item())
        mt["exact_hits"] += int(hit.sum().item())
        mt["exact_inserts"] += int((novel & keep).sum().item())
        mt["exact_overwrites"] += int(ow.sum().item())
        mt["exact_fill_ratio"] = float(new_used.any(dim=0).float().mean().item())

    last = st.mem_last_exact
    cur = last.gather(1, idx.view(B, 1)).squeeze(1)
    last.scatter_(1, idx.view(B, 1), torch.where(keep, pos_e.to(last.dtype), cur).view(B, 1))
    st.mem_last_exact = last

    if trace is not None:
        trace.append(("exact_one", idx.clone(), ow.clone(), keep.clone(), sc.clone()))

    frustrated = int((novel & keep & ~free_exists).any().item())
    if frustrated > 0 and not m.training:
        m._try_expand(st, frustrated, 0)


def summary_one(m, st, k_e, v_e, pos_e, gate, trace=None):
    """Summary bank, one evicted token, memory_banks.py:343-432."""
    if m.Ms == 0:
        return
    B = k_e.shape[0]
    Ms, As, s0, lf = m.Ms, st.active_summary, m.window + m.Me, m.lf_start
    keep = gate >= m.write_gate_threshold_summary if m.write_policy != "none" else torch.ones(B, dtype=torch.bool)
    mem_k = st.k_buf[:, :, s0:]
    mem_v = st.v_buf[:, :, s0:]
    used = st.allowed[:, s0:]

    sc = torch.einsum("bhd,bhmd->bhm", unit(k_e[..., lf:]), st._sum_lf_k_norm).mean(dim=1)
    if As < Ms:
        sc[:, As:] = -1e9
    idx = sc.argmax(dim=-1)

    eta = torch.sigmoid(m.summary_eta_logit).to(dtype=mem_k.dtype)
    eta = eta.view(1, m.num_kv_heads, 1, 1).expand(B, m.num_kv_heads, 1, 1)
    if m.write_policy != "none":
        eta = eta * gate.to(mem_k.dtype).view(B, 1, 1, 1)
    is_new = None
    if m.summary_overwrite_on_insert:
        is_new = ~used.gather(1, idx.view(B, 1)).squeeze(1)
        eta = torch.where(is_new.view(B, 1, 1, 1), torch.ones_like(eta), eta)
    eta = eta * keep.to(eta.dtype).view(B, 1, 1, 1)

    w = torch.zeros((B, Ms), dtype=mem_k.dtype)
    w.scatter_(1, idx.view(B, 1), 1.0)
    w4 = w[:, None, :, None]
    dk = torch.zeros_like(mem_k)
    dk[..., lf:] = k_e[..., lf:].unsqueeze(2) * m.energy_scale - mem_k[..., lf:]
    new_k = mem_k + eta * w4 * dk
    new_v = mem_v + eta * w4 * (v_e.unsqueeze(2) - mem_v)
    new_used = used | (keep.view(B, 1) & w.to(torch.bool))
    st.k_buf[:, :, s0:] = new_k
    st.v_buf[:, :, s0:] = new_v
    st.allowed[:, s0:] = new_used
    st._sum_lf_k_norm = unit(new_k[..., lf:])

    if trace is not None:
        trace.append(("summary_one", idx.clone(), keep.clone(), sc.clone()))

    frustrated = int((new_used[:, :As].all() & keep.any()).item())
    if frustrated > 0 and not m.training:
        m._try_expand(st, 0, frustrated)
    if st.metrics is not None:
        mt = st.metrics
        mt["summary_updates"] += int(keep.sum().item())
        mt["summary_frustrated"] += frustrated
        if m.summary_overwrite_on_insert:
            mt["summary_inserts"] += int((is_new & keep).sum().item())
        mt["summary_fill_ratio"] = float(new_used.any(dim=0).float().mean().item())


# --------------------------------------------------------------------------
# prefill: one block
# --------------------------------------------------------------------------

def _summary_weights(m, vals, dtype):
    """Gate -> summary weight (zero below threshold), memory_banks.py:518-523."""
    w = vals.to(dtype=dtype)
    if m.write_policy != "none":
        w = torch.where(vals >= m.write_gate_threshold_summary, w, torch.zeros_like(w))
    return w


def write_block(m, st, k_blk, v_blk, g_blk, pos0, trace=None):
    """Evict / select candidates / update banks / rebuild ring, memory_banks.py:438-564."""
    B, Hkv, blk, Dh = k_blk.shape
    W = m.window
    k_old, v_old, g_old = ring_time_order(m, st)
    Lr = k_old.shape[2]
    k_cat = torch.cat([k_old, k_blk], dim=2)
    v_cat = torch.cat([v_old, v_blk], dim=2)
    g_cat = torch.cat([g_old, g_blk.to(torch.float32)], dim=1)
    total = Lr + blk
    keep_len = min(W, total)
    n_ev = total - keep_len
    if st.metrics is not None and n_ev > 0:
        st.metrics["total_evictions"] += n_ev

    if n_ev > 0:
        k_e, v_e, g_e = k_cat[:, :, :n_ev].detach(), v_cat[:, :, :n_ev].detach(), g_cat[:, :n_ev].detach()
        pos_e = (torch.arange(n_ev, dtype=torch.int64).view(1, n_ev) + int(pos0 - Lr)).expand(B, n_ev)
        do_e = m.Me > 0 and m.exact_candidates_per_block > 0
        do_s = m.Ms > 0 and m.summary_candidates_per_block > 0

        def pick(T):
            vals, ids = torch.topk(g_e, k=T, dim=1, largest=True, sorted=False)
            ix = ids.view(B, 1, T, 1).expand(B, Hkv, T, Dh)
            return vals, ids, k_e.gather(2, ix), v_e.gather(2, ix), pos_e.gather(1, ids)

        if do_e and do_s:
            Te = min(m.exact_candidates_per_block, n_ev)
            Ts = min(m.summary_candidates_per_block, n_ev)
            vals, ids, ks, vs, ps = pick(max(Te, Ts))
            if trace is not None:
                trace.append(("select", ids.clone()))
            vn = unit(vs)
            kn = unit(ks[..., m.lf_start:])
            exact_block(m, st, ks[:, :, :Te], vs[:, :, :Te], ps[:, :Te], vals[:, :Te], vn[:, :, :Te], trace)
            summary_block(m, st, ks[:, :, :Ts], vs[:, :, :Ts], ps[:, :Ts],
                          _summary_weights(m, vals[:, :Ts], ks.dtype), kn[:, :, :Ts], trace)
        elif do_e:
            vals, ids, ks, vs, ps = pick(min(m.exact_candidates_per_block, n_ev))
            if trace is not None:
                trace.append(("select", ids.clone()))
            exact_block(m, st, ks, vs, ps, vals, None, trace)
        elif do_s:
            vals, ids, ks, vs, ps = pick(min(m.summary_candidates_per_block, n_ev))
            if trace is not None:
                trace.append(("select", ids.clone()))
            summary_block(m, st, ks, vs, ps, _summary_weights(m, vals, ks.dtype), None, trace)

    lo = total - keep_len
    ring_rebuild(m, st, k_cat[:, :, lo:total], v_cat[:, :, lo:total], g_cat[:, lo:total])
    st.pos = int(pos0 + blk)


def exact_block(m, st, k_sel, v_sel, pos_sel, gate_sel, v_sel_norm=None, trace=None):
    """Exact bank, T candidates, PyTorch branch of memory_banks.py:570-774."""
    if m.Me == 0:
        return
    B, Hkv, T, Dh = k_sel.shape
    Me, Ae, W = m.Me, st.active_exact, m.window
    mem_k = st.k_buf[:, :, W:W + Me]
    mem_v = st.v_buf[:, :, W:W + Me]
    used = st.allowed[:, W:W + Me]
    last = st.mem_last_exact
    if v_sel_norm is None:
        v_sel_norm = unit(v_sel)

    keep = gate_sel >= m.write_gate_threshold_exact if m.write_policy != "none" else torch.ones((B, T), dtype=torch.bool)
    sc = torch.matmul(v_sel_norm.reshape(B * Hkv, T, Dh),
                      st._exact_v_norm.reshape(B * Hkv, Me, Dh).transpose(1, 2)).view(B, Hkv, T, Me).mean(dim=1)
    if Ae < Me:
        sc.masked_fill_((torch.arange(Me).unsqueeze(0) >= Ae).unsqueeze(1), -1e9)
    sc.masked_fill_(~used[:, None, :], -1e9)
    best, best_idx = sc.max(dim=-1)
    any_used = used.any(dim=-1)
    novel = (~any_used[:, None]) | (best < m.exact_novelty_threshold)
    hit = any_used[:, None] & (best >= m.exact_match_threshold)
    nk = novel & keep

    rk = last.clone()
    rk[~used] = NEG_BIG
    if Ae < Me:
        rk[:, Ae:] = NEG_BIG
    n_lru = min(T, Ae)
    _, lru = torch.topk(rk, k=n_lru, dim=1, largest=False, sorted=True)
    rank = nk.to(torch.int64).cumsum(dim=1) - 1
    cap = nk & (rank < Ae)
    slot = lru.gather(1, rank.clamp(min=0, max=max(n_lru - 1, 0)))
    idx = torch.where(cap, slot, best_idx)
    touch = keep & (~novel | cap)
    ow = keep & (cap | hit) if m.exact_refresh_on_hit else cap

    tmask = torch.zeros((B, Me), dtype=torch.int8)
    tmask.scatter_reduce_(1, idx, touch.to(torch.int8), reduce="amax", include_self=True)
    pv = torch.full((B, Me), NEG_BIG, dtype=pos_sel.dtype)
    pv.scatter_reduce_(1, idx, torch.where(touch, pos_sel, torch.full_like(pos_sel, NEG_BIG)),
                       reduce="amax", include_self=True)
    st.mem_last_exact = torch.where(tmask.to(torch.bool), pv, last)

    ix = idx.unsqueeze(1).unsqueeze(-1).expand(B, Hkv, T, Dh)
    owf = ow.to(dtype=mem_k.dtype).view(B, 1, T, 1)
    dk = owf * (k_sel - mem_k.gather(2, ix))
    dv = owf * (v_sel - mem_v.gather(2, ix))
    new_k = mem_k + torch.zeros_like(mem_k).scatter_add_(2, ix, dk)
    new_v = mem_v + torch.zeros_like(mem_v).scatter_add_(2, ix, dv)
    smask = torch.zeros((B, Me), dtype=torch.int8)
    smask.scatter_reduce_(1, idx, ow.to(torch.int8), reduce="amax", include_self=True)
    smask = smask.to(torch.bool)
    new_used = used | smask
    st.k_buf[:, :, W:W + Me] = new_k
    st.v_buf[:, :, W:W + Me] = new_v
    st.allowed[:, W:W + Me] = new_used
    changed = smask.any(dim=0).nonzero(as_tuple=True)[0]
    st._exact_v_norm[:, :, changed, :] = unit(new_v[:, :, changed, :])

    if trace is not None:
        trace.append(("exact_block", idx.clone(), ow.clone(), touch.clone(), sc.clone()))

    frustrated = int((nk & ~cap).sum().item())
    if frustrated > 0 and not m.training:
        m._try_expand(st, frustrated, 0)
    if st.metrics is not None:
        mt = st.metrics
        mt["exact_overwrites"] += int(ow.sum().item())
        mt["exact_frustrated"] += frustrated
        mt["exact_fill_ratio"] = float(new_used.any(dim=0).float().mean().item())
        mt["exact_inserts"] += int(cap.sum().item())
        mt["exact_hits"] += int((hit & keep).sum().item())
        if m.write_policy != "none":
            mt["tokens_gated_out"] += int((~keep).sum().item())


def summary_block(m, st, k_sel, v_sel, pos_sel, w_tok, lf_k_sel_norm=None, trace=None):
    """Summary bank, T candidates, PyTorch branch of memory_banks.py:780-950."""
    if m.Ms == 0:
        return
    B, Hkv, T, Dh = k_sel.shape
    Ms, As, s0, lf = m.Ms, st.active_summary, m.window + m.Me, m.lf_start
    mem_k = st.k_buf[:, :, s0:]
    mem_v = st.v_buf[:, :, s0:]
    used = st.allowed[:, s0:]
    if lf_k_sel_norm is None:
        lf_k_sel_norm = unit(k_sel[..., lf:])
    sc = torch.matmul(lf_k_sel_norm.reshape(B * Hkv, T, Dh - lf),
                      st._sum_lf_k_norm.reshape(B * Hkv, Ms, Dh - lf).transpose(1, 2)).view(B, Hkv, T, Ms).mean(dim=1)
    if As < Ms:
        sc.masked_fill_((torch.arange(Ms).unsqueeze(0) >= As).unsqueeze(1), -1e9)
    idx = sc.argmax(dim=-1)

    dt = mem_k.dtype
    w = w_tok.to(dtype=dt)
    count = torch.zeros(B, Ms, dtype=dt).scatter_add_(1, idx, w)
    ix = idx.unsqueeze(1).unsqueeze(-1).expand(B, Hkv, T, Dh)
    w4 = w.view(B, 1, T, 1)
    sum_k = torch.zeros(B, Hkv, Ms, Dh, dtype=dt).scatter_add_(2, ix, k_sel * w4)
    sum_v = torch.zeros(B, Hkv, Ms, Dh, dtype=dt).scatter_add_(2, ix, v_sel * w4)

    eta = torch.sigmoid(m.summary_eta_logit).to(dtype=dt).view(1, Hkv, 1, 1)
    c4 = count.view(B, 1, Ms, 1)
    active = c4 > 0
    avg_k = sum_k / c4.clamp_min(1e-6)
    avg_v = sum_v / c4.clamp_min(1e-6)
    fresh = (~used).view(B, 1, Ms, 1) & active
    eta_eff = torch.where(fresh, torch.ones_like(eta), eta) if m.summary_overwrite_on_insert else eta
    dk = torch.zeros_like(avg_k)
    dk[..., lf:] = avg_k[..., lf:] * m.energy_scale - mem_k[..., lf:]
    new_k = torch.where(active, mem_k + eta_eff * dk, mem_k)
    new_v = torch.where(active, mem_v + eta_eff * (avg_v - mem_v), mem_v)
    new_used = used | (count > 0)
    st.k_buf[:, :, s0:] = new_k
    st.v_buf[:, :, s0:] = new_v
    st.allowed[:, s0:] = new_used
    touched = (count > 0).any(dim=0).nonzero(as_tuple=True)[0]
    if touched.numel() > 0:
        st._sum_lf_k_norm[:, :, touched, :] = unit(new_k[:, :, touched, lf:])

    if trace is not None:
        trace.append(("summary_block", idx.clone(), sc.clone()))

    frustrated = int(new_used[:, :As].all().item() and (count[:, :As] > 0).any().item())
    if frustrated > 0 and not m.training:
        m._try_expand(st, 0, frustrated)
    if st.metrics is not None:
        mt = st.metrics
        mt["summary_updates"] += int((count > 0).sum().item())
        mt["summary_frustrated"] += frustrated
        if m.summary_overwrite_on_insert:
            mt["summary_inserts"] += int(fresh.sum().item())
        mt["summary_fill_ratio"] = float(new_used.any(dim=0).float().mean().item())
