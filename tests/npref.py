"""Independent numpy restatements used to pin the C oracle.

These decode the GGUF block formats with vectorized bit arithmetic written from
the format definitions (not from the oracle's loops), and compute reductions in
float64, so a dropped term, wrong index, sign or transposed operand in the
oracle shows up as a mismatch.
"""
import numpy as np


def f16_to_f32(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def deq_q8_0(row, n):
    b = np.asarray(row, np.uint8).reshape(-1, 34)[: n // 32]
    d = f16_to_f32(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).reshape(-1)


def _k4_scales(sc):
    """6-bit scales/mins of a Q4_K block (12 bytes) -> (8,), (8,) uint8."""
    sc = sc.astype(np.int32)
    s = np.zeros(sc.shape[:-1] + (8,), np.int32)
    m = np.zeros_like(s)
    s[..., :4] = sc[..., 0:4] & 63
    m[..., :4] = sc[..., 4:8] & 63
    s[..., 4:] = (sc[..., 8:12] & 0xF) | ((sc[..., 0:4] >> 6) << 4)
    m[..., 4:] = (sc[..., 8:12] >> 4) | ((sc[..., 4:8] >> 6) << 4)
    return s, m


def deq_q4_k(row, n):
    b = np.asarray(row, np.uint8).reshape(-1, 144)[: n // 256]
    d = f16_to_f32(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    dm = f16_to_f32(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    s, m = _k4_scales(b[:, 4:16])
    qs = b[:, 16:].reshape(-1, 4, 32)
    nib = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)
    d1 = (d[:, None] * s.astype(np.float32))[:, :, None]
    m1 = (dm[:, None] * m.astype(np.float32))[:, :, None]
    return (d1 * nib - m1).astype(np.float32).reshape(-1)


def q6_k_ints(row, n):
    """Q6_K block -> signed 6-bit values (nb,256) int32 and int8 scales (nb,16)."""
    b = np.asarray(row, np.uint8).reshape(-1, 210)[: n // 256]
    ql = b[:, 0:128].reshape(-1, 2, 64).astype(np.int32)
    qh = b[:, 128:192].reshape(-1, 2, 32).astype(np.int32)
    q = np.zeros((b.shape[0], 2, 128), np.int32)
    q[:, :, 0:32] = (ql[:, :, 0:32] & 0xF) | ((qh & 3) << 4)
    q[:, :, 32:64] = (ql[:, :, 32:64] & 0xF) | (((qh >> 2) & 3) << 4)
    q[:, :, 64:96] = (ql[:, :, 0:32] >> 4) | (((qh >> 4) & 3) << 4)
    q[:, :, 96:128] = (ql[:, :, 32:64] >> 4) | (((qh >> 6) & 3) << 4)
    sc = b[:, 192:208].view(np.int8).astype(np.int32)
    d = f16_to_f32(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
    return (q - 32).reshape(-1, 256), sc, d


def deq_q6_k(row, n):
    q, sc, d = q6_k_ints(row, n)
    s_per = np.repeat(sc, 16, axis=1).astype(np.float32)  # element i uses scale i//16
    return ((d[:, None] * s_per) * q.astype(np.float32)).astype(np.float32).reshape(-1)


MXFP4_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                        np.float32)


def deq_mxfp4(row, n):
    b = np.asarray(row, np.uint8).reshape(-1, 17)[: n // 32]
    scale = np.ldexp(np.float32(1.0), b[:, 16].astype(np.int32) - 127).astype(np.float32)
    nib = np.stack([b[:, :16] & 0xF, b[:, :16] >> 4], axis=2).reshape(-1, 32)
    return (MXFP4_VALUES[nib] * scale[:, None]).astype(np.float32).reshape(-1)


DEQ = {8: deq_q8_0, 12: deq_q4_k, 14: deq_q6_k, 39: deq_mxfp4}


def q8k(x):
    """Q8_K closed form: per 256, d = amax*(1/127), q = clamp(rne(x*(127/amax)))."""
    x = np.asarray(x, np.float32).reshape(-1, 256)
    amax = np.abs(x).max(axis=1)
    d = (amax * np.float32(1.0 / 127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint((x * idv[:, None]).astype(np.float32)), -128, 127).astype(np.int8)
    bs = q.reshape(-1, 8, 32).astype(np.int32).sum(axis=2).astype(np.int16).reshape(-1)
    return q.reshape(-1), d, bs


def attention_f64(q, K, V, n_heads, n_kv, hd, vd, scale, sinks=None):
    """Textbook softmax(q.K^T * scale).V in float64 over an already-gathered
    context K (T, n_kv*hd), V (T, n_kv*vd); sinks add one logit with zero value."""
    q = np.asarray(q, np.float64).reshape(n_heads, hd)
    K = np.asarray(K, np.float64).reshape(-1, n_kv, hd)
    V = np.asarray(V, np.float64).reshape(-1, n_kv, vd)
    kv_mul = n_heads // n_kv
    out = np.zeros((n_heads, vd))
    for h in range(n_heads):
        s = K[:, h // kv_mul, :] @ q[h] * float(scale)
        m = s.max()
        if sinks is not None:
            m = max(m, float(sinks[h]))
        w = np.exp(s - m)
        den = w.sum() + (np.exp(float(sinks[h]) - m) if sinks is not None else 0.0)
        out[h] = (w @ V[:, h // kv_mul, :]) / den
    return out.reshape(-1)


def deq_matrix(w, t, rows, cols):
    if t == 0:
        return np.asarray(w).view(np.float32).reshape(rows, cols).astype(np.float64)
    return DEQ[t](w, rows * cols).reshape(rows, cols).astype(np.float64)


def q8k_dequant(x):
    q, d, _ = q8k(np.asarray(x, np.float32))
    return (q.astype(np.float64).reshape(-1, 256) * d.astype(np.float64)[:, None]).reshape(-1)


def matvec_ref(w, t, rows, cols, x):
    """Integer Q8_K paths equal dequant(W) . dequant(q8k(x)) exactly in real
    arithmetic (the block formula factors per element); f32 paths use x."""
    W = deq_matrix(w, t, rows, cols)
    int_path = t in (12, 14) or (t == 8 and cols % 256 == 0)
    xv = q8k_dequant(x) if int_path else np.asarray(x, np.float64)
    return W @ xv


def bf16_round(x):
    """x through a bf16 store: f32, round to nearest even on the top 16 bits."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFFFFFF) >> 16 << 16).astype(np.uint32)
    return r.view(np.float32).astype(np.float64)


def forward_model(model, tokens, start_pos=0, kv_bf16=False):
    """float64 restatement of forward_into (src/model.rs:7177-7358) for a
    rustyllm_amd.synth model; returns the logits of every position.  kv_bf16:
    the cache keeps each K/V element as its bf16 rounding (KVCache::write_k /
    write_v with enable_bf16)."""
    c = model["config"]
    dim, hd, vd = c["dim"], c["head_dim"], c.get("value_dim", c["head_dim"])
    nh, nkv = c["n_heads"], c["n_kv_heads"]
    kv_mul = nh // nkv
    eps = c["eps"]
    inv = np.asarray(model["inv_freq"], np.float32)
    neox = c.get("neox", False)
    emb_w, emb_t = model["token_embd"]
    E = deq_matrix(emb_w, emb_t, c["vocab"], dim)
    Ws = [[deq_matrix(a, t, r, (dim if i not in (3, 6) else (nh * vd if i == 3 else c["hidden_dim"])))
           for i, (a, t, r) in enumerate(L["w"])] for L in model["layers"]]
    out_w, out_t = model["output"]
    Wo = deq_matrix(out_w, out_t, c["vocab"], dim)
    K = [[] for _ in model["layers"]]
    V = [[] for _ in model["layers"]]
    logits_all = []

    def rms(x, w):
        return x / np.sqrt((x * x).mean() + eps) * w

    def mv(W, i, x, L, cols):
        a, t, r = model["layers"][L]["w"][i]
        int_path = t in (12, 14) or (t == 8 and cols % 256 == 0)
        xv = q8k_dequant(x) if int_path else x
        return W @ xv

    def rope(x, n, pos):
        x = x.reshape(n, hd).copy()
        ang = (np.float32(pos) * inv).astype(np.float64)
        cs, sn = np.cos(ang), np.sin(ang)
        if neox:
            a, b = x[:, :hd // 2].copy(), x[:, hd // 2:].copy()
            x[:, :hd // 2], x[:, hd // 2:] = a * cs - b * sn, a * sn + b * cs
        else:
            a, b = x[:, 0::2].copy(), x[:, 1::2].copy()
            x[:, 0::2], x[:, 1::2] = a * cs - b * sn, a * sn + b * cs
        return x.reshape(-1)

    for ti, tok in enumerate(tokens):
        pos = start_pos + ti
        x = E[tok].copy()
        for l, L in enumerate(model["layers"]):
            W = Ws[l]
            xn = rms(x, L["attn_norm"].astype(np.float64))
            q = mv(W[0], 0, xn, l, dim)
            k = mv(W[1], 1, xn, l, dim)
            v = mv(W[2], 2, xn, l, dim)
            if L.get("bq") is not None:
                q, k, v = q + L["bq"], k + L["bk"], v + L["bv"]
            q, k = rope(q, nh, pos), rope(k, nkv, pos)
            K[l].append(bf16_round(k) if kv_bf16 else k)
            V[l].append(bf16_round(v) if kv_bf16 else v)
            Kc, Vc = np.array(K[l]), np.array(V[l])
            att = attention_f64(q, Kc, Vc, nh, nkv, hd, vd, np.float32(1.0) / np.sqrt(np.float32(hd)))
            x = x + mv(W[3], 3, att, l, nh * vd)
            xn = rms(x, L["ffn_norm"].astype(np.float64))
            g = mv(W[4], 4, xn, l, dim)
            u = mv(W[5], 5, xn, l, dim)
            h = g / (1 + np.exp(-g)) * u
            x = x + mv(W[6], 6, h, l, c["hidden_dim"])
        xn = rms(x, model["output_norm"].astype(np.float64))
        int_path = out_t in (12, 14) or (out_t == 8 and dim % 256 == 0)
        logits_all.append(Wo @ (q8k_dequant(xn) if int_path else xn))
    return np.array(logits_all)


def forward_gptoss(model, tokens, max_len, ring=True):
    """float64 restatement of forward_gpt_oss_into (src/model.rs:6733-6908)
    for a rustyllm_amd.synth.make_gptoss model; returns every position's
    logits.  Written from the semantics, not the oracle's loops:
    - the KV cache is a ring of S = min(window, max_len) slots
      (KVCache::with_sliding_window, model.rs:1363-1385); after position pos
      is stored, slot s holds the newest position p <= pos with p % S == s;
    - every layer scans steps t = start..pos reading slot t % S (the
      reference's incrementing-slot walk), start = pos + 1 - window on even
      layers and 0 on odd ones, so an odd layer past S positions sees each
      slot's newest entry, cyclically, pos + 1 times in all;
    - softmax over those scores plus the head's sink logit (zero value row)."""
    c = model["config"]
    dim, hd, vd = c["dim"], c["head_dim"], c.get("value_dim", c["head_dim"])
    nh, nkv, hid = c["n_heads"], c["n_kv_heads"], c["hidden_dim"]
    W = c["window"]
    # ring=False: a linear cache of max_len slots (for showing that the ring matters)
    S = min(W, max_len) if (W > 0 and ring) else max_len
    kv_mul = nh // nkv
    eps, conc, inv = c["eps"], float(model["concentration"]), np.asarray(model["inv_freq"], np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    emb_w, emb_t = model["token_embd"]
    E = deq_matrix(emb_w, emb_t, c["vocab"], dim)
    out_w, out_t = model["output"]
    Wout = deq_matrix(out_w, out_t, c["vocab"], dim)
    ne = c["n_experts"]

    def mv(Wm, x, t, cols):
        int_path = t in (12, 14) or (t == 8 and cols % 256 == 0)
        return Wm @ (q8k_dequant(x) if int_path else x)

    def rms(x, w):
        return x / np.sqrt((x * x).mean() + eps) * np.asarray(w, np.float64)

    def rope(x, n, pos):
        x = x.reshape(n, hd).copy()
        ang = (np.float32(pos) * inv).astype(np.float64)
        cs, sn = np.cos(ang) * conc, np.sin(ang) * conc
        a, b = x[:, 0::2].copy(), x[:, 1::2].copy()
        x[:, 0::2], x[:, 1::2] = a * cs - b * sn, a * sn + b * cs
        return x.reshape(-1)

    def swiglu(g, u):
        g = np.minimum(g, 7.0)
        u = np.clip(u, -7.0, 7.0)
        return g / (1.0 + np.exp(-1.702 * g)) * (u + 1.0)

    layers = []
    for L in model["layers"]:
        D = {nm: deq_matrix(L[nm][0], L[nm][1], r, cl) for nm, r, cl in
             (("wq", nh * hd, dim), ("wk", nkv * hd, dim), ("wv", nkv * vd, dim), ("wo", dim, nh * vd))}
        D["router"] = deq_matrix(L["router"], 8, ne, dim)
        D["gate"] = deq_matrix(L["gate_exps"], 39, ne * hid, dim).reshape(ne, hid, dim)
        D["up"] = deq_matrix(L["up_exps"], 39, ne * hid, dim).reshape(ne, hid, dim)
        D["down"] = deq_matrix(L["down_exps"], 39, ne * dim, hid).reshape(ne, dim, hid)
        layers.append(D)
    hist_k = [[] for _ in layers]
    hist_v = [[] for _ in layers]
    logits_all = []
    for pos, tok in enumerate(tokens):
        x = E[tok].copy()
        for l, (L, D) in enumerate(zip(model["layers"], layers)):
            xn = rms(x, L["attn_norm"])
            q = mv(D["wq"], xn, L["wq"][1], dim) + L["bq"]
            k = mv(D["wk"], xn, L["wk"][1], dim) + L["bk"]
            v = mv(D["wv"], xn, L["wv"][1], dim) + L["bv"]
            q, k = rope(q, nh, pos), rope(k, nkv, pos)
            hist_k[l].append(k.reshape(nkv, hd))
            hist_v[l].append(v.reshape(nkv, vd))
            start = max(0, pos + 1 - W) if (l % 2 == 0 and W > 0) else 0
            steps = np.arange(start, pos + 1)
            slots = steps % S if W > 0 else steps
            # newest position stored in each slot by now
            newest = pos - ((pos - slots) % S) if W > 0 else slots
            Kc = np.array([hist_k[l][p] for p in newest])
            Vc = np.array([hist_v[l][p] for p in newest])
            qh = q.reshape(nh, hd)
            att = np.zeros((nh, vd))
            for h in range(nh):
                s = Kc[:, h // kv_mul, :] @ qh[h] * scale
                sink = float(L["sinks"][h])
                m = max(s.max(), sink)
                w = np.exp(s - m)
                att[h] = (w @ Vc[:, h // kv_mul, :]) / (w.sum() + np.exp(sink - m))
            x = x + mv(D["wo"], att.reshape(-1), L["wo"][1], nh * vd) + L["bo"]
            xn2 = rms(x, L["post_attn_norm"])
            r = mv(D["router"], xn2, 8, dim) + L["router_bias"]
            sel = np.argsort(-r, kind="stable")[: c["top_k"]]
            p = np.exp(r[sel] - r[sel].max())
            p /= p.sum()
            moe = np.zeros(dim)
            for e, pe in zip(sel, p):
                g = D["gate"][e] @ xn2 + L["gate_exps_bias"][e]
                u = D["up"][e] @ xn2 + L["up_exps_bias"][e]
                moe += (D["down"][e] @ swiglu(g, u) + L["down_exps_bias"][e]) * pe
            x = x + moe
        xn = rms(x, model["output_norm"])
        logits_all.append(mv(Wout, xn, out_t, dim))
    return np.array(logits_all)
