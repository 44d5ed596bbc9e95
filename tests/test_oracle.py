"""Pins the CPU oracle (oracle/eager.py) with checks that do not restate its
formulas: float64 brute force, exhaustive enumeration, format definitions,
known answers from the reference's own tests and invariants."""
import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import eager as O


def brute_rmsnorm_linear(x, W, b=None, eps=1e-6, scale=1.0, gamma=None, norm=True):
    x = np.asarray(x, dtype=np.float64)
    W = np.asarray(W, dtype=np.float64)
    M, K = x.shape
    N = W.shape[0]
    y = np.zeros((M, N))
    for m in range(M):
        ss = sum(v * v for v in x[m])
        rs = 1.0 / math.sqrt(ss / K + eps) if norm else 1.0
        xn = [x[m, k] * rs * (gamma[k] if gamma is not None else 1.0) for k in range(K)]
        for n in range(N):
            acc = sum(xn[k] * W[n, k] for k in range(K))
            if b is not None:
                acc += b[n]
            y[m, n] = acc * scale
    return y


def test_rmsnorm_linear_matches_fp64_brute_force():
    # Same seeded inputs as the reference's check (test_engine.py:5).
    torch.manual_seed(1)
    x = torch.randn(5, 64)
    W = torch.randn(128, 64)
    b = torch.randn(128)
    y = O.rmsnorm_linear(x, W, b, 1e-6)
    ref = brute_rmsnorm_linear(x.numpy(), W.numpy(), b.numpy())
    assert np.abs(y.numpy() - ref).max() < 1e-4  # the reference's bound
    assert np.abs(y.numpy() - ref).max() / np.abs(ref).max() < 1e-6


def test_rmsnorm_linear_gamma_scale_nonorm_brute_force():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 24, generator=g)
    W = torch.randn(10, 24, generator=g)
    gamma = 1 + 0.1 * torch.randn(24, generator=g)
    for norm in (True, False):
        y = O.rmsnorm_linear(x, W, None, 1e-6, 0.5, gamma=gamma, norm=norm)
        ref = brute_rmsnorm_linear(x.numpy(), W.numpy(), None, 1e-6, 0.5, gamma.numpy(), norm)
        assert np.allclose(y.numpy(), ref, rtol=1e-5, atol=1e-6)


def test_rmsnorm_linear_invariants():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 256, generator=g)
    W = torch.randn(32, 256, generator=g)
    y1 = O.rmsnorm_linear(x, W, None, 0.0)
    y2 = O.rmsnorm_linear(3.7 * x, W, None, 0.0)
    assert torch.allclose(y1, y2, rtol=1e-5, atol=1e-5)  # RMSNorm is scale invariant
    assert torch.equal(O.rmsnorm_linear(x, W, None, 1e-6, gamma=torch.ones(256)),
                       O.rmsnorm_linear(x, W, None, 1e-6))


def test_bias_is_cast_to_x_dtype():
    # The wrapper casts bias to x.dtype before the fp32 linear (mtp_kernels.py:952).
    x = torch.randn(2, 16).to(torch.bfloat16)
    W = torch.randn(8, 16)
    b = torch.full((8,), 1.0 + 2.0 ** -12)  # not representable in bf16
    y = O.rmsnorm_linear(x, W, b, 1e-6).float()
    y0 = O.rmsnorm_linear(x, W, torch.ones(8), 1e-6).float()
    assert torch.equal(y, y0)
    assert y.dtype == torch.float32 and O.rmsnorm_linear(x, W, b).dtype == torch.bfloat16


def test_fp8_decode_table_matches_torch_cast():
    table = O.fp8_e4m3fn_decode_table()
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    nan = np.isnan(table)
    assert np.array_equal(nan, np.isnan(vals))
    assert np.array_equal(table[~nan], vals[~nan])
    assert np.nanmax(table) == 448.0 and nan.sum() == 2


def test_fp8_per_channel_quantizer():
    g = torch.Generator().manual_seed(11)
    W = 0.02 * torch.randn(6, 512, generator=g)
    W[3] = 0.0
    q, s = O.quantize_fp8_per_channel(W)
    amax = np.abs(W.numpy()).max(axis=1)
    exp_s = np.where(amax > 0, amax / np.float32(448.0), 1.0).astype(np.float32)
    assert np.array_equal(s.numpy(), exp_s)
    v = (W / s[:, None]).numpy().astype(np.float64)
    qv = q.to(torch.float64).numpy()
    # spacing of e4m3 at |v|: 2^(floor(log2|v|) - 3), subnormal spacing 2^-9
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -6)))
    spacing = 2.0 ** (e - 3)
    assert (np.abs(v - qv) <= spacing / 2 + 1e-12).all()
    assert np.abs(qv).max() <= 448.0
    assert (qv[3] == 0).all()


def test_rmsnorm_linear_fp8_brute_force():
    g = torch.Generator().manual_seed(5)
    W = torch.randn(16, 32, generator=g)
    q, s = O.quantize_fp8_per_channel(W)
    x = torch.randn(3, 32, generator=g)
    table = O.fp8_e4m3fn_decode_table()
    wd = table[q.view(torch.uint8).numpy().astype(np.int64)] * s.numpy()[:, None].astype(np.float64)
    ref = brute_rmsnorm_linear(x.numpy(), wd)
    y = O.rmsnorm_linear_fp8(x, q, s)
    assert np.abs(y.numpy() - ref).max() < 1e-4 * max(1.0, np.abs(ref).max())


def test_int4_decode_all_bytes():
    packed = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(1, 256)
    w = O.dequantize_int4(packed, torch.ones(1, 1), 512, 512)
    exp = []
    for b in range(256):
        exp += [(b & 0xF) - 8, ((b >> 4) & 0xF) - 8]
    assert w.numpy().tolist() == [exp]
    w2 = O.dequantize_int4(packed, torch.ones(1, 1), 512, 512, nibble="twos")
    tw = []
    for b in range(256):
        lo, hi = b & 0xF, b >> 4
        tw += [lo - 16 if lo >= 8 else lo, hi - 16 if hi >= 8 else hi]
    assert w2.numpy().tolist() == [tw]


def test_int4_pack_order_and_reference_roundtrip_mismatch():
    # Exact multiples of the group scale: q = +1 on even k, -3 on odd k.
    K, group = 64, 32
    q = np.tile([1, -3], K // 2).astype(np.float32)
    q[5] = 7.0  # sets the group amax -> scale = 1
    q[37] = -7.0
    W = torch.from_numpy(q[None, :].copy())
    packed, scales = O.quantize_int4(W, group)
    assert torch.equal(scales, torch.ones(1, 2))
    assert int(packed[0, 0]) == ((1 & 0xF) | ((-3 & 0xF) << 4))  # even k -> low nibble
    back = O.dequantize_int4(packed, scales, K, group).numpy()[0]
    exp = np.where(q >= 0, q - 8, q + 8)  # the reference's pack/unpack disagree
    assert np.array_equal(back, exp)
    packed_o, _ = O.quantize_int4(W, group, nibble="offset")
    assert np.array_equal(O.dequantize_int4(packed_o, scales, K, group).numpy()[0], q)


def test_int4_quantizer_rounds_half_to_even():
    """Planted half-integer ties of W / s with literal expected values: the
    reference rounds with torch.round (mtp_kernels.py:745), i.e. half to
    even: 2.5 -> 2, 3.5 -> 4, -2.5 -> -2, 0.5 -> 0, -0.5 -> 0, 1.5 -> 2,
    -1.5 -> -2, 4.5 -> 4, 5.5 -> 6, -3.5 -> -4; amax 7 fixes s = 1. A
    quantizer rounding half away from zero, or truncating, fails here."""
    K, group = 32, 32
    vals = [2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -1.5, 4.5, 5.5, -3.5, 7.0, 6.5, -6.5, -7.0]
    exp_q = [2, 4, -2, 0, 0, 2, -2, 4, 6, -4, 7, 6, -6, -7]
    row = np.zeros(K, dtype=np.float32)
    row[:len(vals)] = vals
    packed, scales = O.quantize_int4(torch.from_numpy(row[None, :].copy()), group)
    assert float(scales[0, 0]) == 1.0
    nib = O.int4_nibbles(packed)[0]
    assert nib[:len(vals)].tolist() == [q & 0xF for q in exp_q]          # reference bytes
    po, _ = O.quantize_int4(torch.from_numpy(row[None, :].copy()), group, nibble="offset")
    assert O.int4_nibbles(po)[0][:len(vals)].tolist() == [q + 8 for q in exp_q]
    # literal bytes of the first pairs: (2, 4) and (-2, 0)
    assert int(packed[0, 0]) == 0x42 and int(packed[0, 1]) == 0x0E


def test_int4_matmul_equals_dequant_linear():
    # The reference's own check (mtp_engine.py:1812-1819): bit-identical.
    torch.manual_seed(0)
    W = torch.randn(32, 64)
    pk, sc = O.quantize_int4(W, 32)
    x = torch.randn(4, 64)
    assert torch.equal(O.int4_matmul(x, pk, sc, 64, 32), F.linear(x, O.dequantize_int4(pk, sc, 64, 32)))


def brute_argmax(vals):
    best, bi = None, 0
    for i, v in enumerate(vals):
        if best is None:
            best, bi = v, i
            continue
        if math.isnan(best):
            continue
        if math.isnan(v) or v > best:
            best, bi = v, i
    return bi


def test_verify_brute_force_ties_nan():
    rng = np.random.default_rng(0)
    h = rng.integers(-3, 4, size=(6, 5)).astype(np.float32)
    W = rng.integers(-3, 4, size=(9, 5)).astype(np.float32)
    W[7] = W[2]  # planted tie: index 2 must win over 7
    b = np.zeros(9, dtype=np.float32)
    draft = torch.tensor([0, 1, 2, 3, 4, 5])
    acc, top = O.fused_verify(torch.from_numpy(h), torch.from_numpy(W), draft, torch.from_numpy(b))
    for m in range(6):
        logits = [float(sum(float(h[m, k]) * float(W[v, k]) for k in range(5))) for v in range(9)]
        assert int(top[m]) == brute_argmax(logits)
        assert int(acc[m]) == int(int(top[m]) == int(draft[m]))
    # all-equal logits -> index 0; a NaN logit wins
    _, t0 = O.fused_verify(torch.zeros(1, 5), torch.zeros(9, 5), torch.zeros(1))
    assert int(t0[0]) == 0
    Wn = torch.zeros(9, 5)
    Wn[4, 0] = float("nan")
    _, tn = O.fused_verify(torch.ones(1, 5), Wn, torch.zeros(1))
    assert int(tn[0]) == 4


def test_verify_chunked_argmax_tie_across_chunks():
    W = torch.zeros(40, 4)
    W[5, 0] = 1.0
    W[33, 0] = 1.0  # same logit in a later chunk: 5 must win
    top, gap = O.logits_top(torch.ones(1, 4), W, chunk=16)
    assert int(top[0]) == 5 and float(gap[0]) == 0.0


def test_reference_fused_verify_check_seeded():
    # test_new_features.py:18-31 on the same seeded CPU inputs, against brute force.
    torch.manual_seed(0)
    M, K, V = 4, 64, 256
    h = torch.randn(M, K)
    W = torch.randn(V, K)
    b = torch.randn(V)
    d = torch.randint(0, V, (M,))
    acc, top = O.fused_verify(h, W, d, b)
    hd, Wd, bd = h.double().numpy(), W.double().numpy(), b.double().numpy()
    for m in range(M):
        logits = Wd @ hd[m] + bd
        assert int(top[m]) == int(np.argmax(logits))


@pytest.mark.parametrize("D", [0, 1, 2, 3, 4])
def test_chain_accept_exhaustive(D):
    for pattern in itertools.product([0, 1], repeat=D):
        top = torch.tensor([[7] + [10 + d for d in range(D)]])
        draft = torch.tensor([[10 + d if pattern[d] else 99 for d in range(D)]])
        acc, n, corr = O.chain_accept(top, draft)
        lead = 0
        while lead < D and pattern[lead]:
            lead += 1
        assert int(n[0]) == lead
        assert acc[0].tolist() == [1] * lead + ([0] * (D - lead))
        assert int(corr[0]) == 7


@pytest.mark.parametrize("D", [0, 1, 2, 3, 4])
def test_chain_accept_textbook_exhaustive(D):
    """Every accept / reject pattern of D drafts against the textbook
    convention: draft d is compared with top[b, d] (the argmax after the
    first d accepted tokens), corrected = top[b, accepted_n]. The tokens are
    chosen so that the reference convention (top[b, d + 1]) would give a
    different answer for every pattern with a match."""
    for pattern in itertools.product([0, 1], repeat=D):
        top = torch.tensor([[10 + s for s in range(D + 1)]])  # top[b, s] = 10 + s
        # a matching draft d is 10 + d; a rejected one is 11 + d, which the
        # reference convention would accept
        draft = torch.tensor([[10 + d if pattern[d] else 11 + d for d in range(D)]])
        acc, n, corr = O.chain_accept_textbook(top, draft)
        lead = 0
        while lead < D and pattern[lead]:
            lead += 1
        assert int(n[0]) == lead
        assert acc[0].tolist() == [1] * lead + [0] * (D - lead)
        assert int(corr[0]) == 10 + lead  # replacement token, or the bonus 10 + D
        racc, rn, rcorr = O.chain_accept(top, draft)
        assert int(rcorr[0]) == 10
        if D and not pattern[0]:
            assert int(rn[0]) >= 1  # the reference convention takes 11 as the first draft


def test_multi_verify_matches_reference_test_seeded():
    # test_new_features.py:34-56 on the same seeded CPU inputs, brute-force logits.
    torch.manual_seed(1)
    B, S, K, V, D = 2, 5, 64, 256, 4
    hidden = torch.randn(B, S, K)
    W = torch.randn(V, K)
    b = torch.randn(V)
    draft = torch.randint(0, V, (B, D))
    acc, n, corr, top, _ = O.fused_multi_verify(hidden, W, draft, b)
    Wd, bd = W.double().numpy(), b.double().numpy()
    for i in range(B):
        t = [int(np.argmax(Wd @ hidden[i, s].double().numpy() + bd)) for s in range(S)]
        assert top[i].tolist() == t
        assert int(corr[i]) == t[0]
        ref_n = 0
        for d in range(D):
            if t[d + 1] == int(draft[i, d]):
                ref_n = d + 1
            else:
                break
        assert int(n[i]) == ref_n


def test_draft_tree_known_shapes():
    parent, mask = O.draft_tree(4, 8, "tree")
    assert mask.shape == (32, 32) and mask[0, 0] == 1.0
    _, tmask = O.draft_tree(4, 8, "trunk")
    assert tmask[1, 0] == 1.0 and tmask[1, 2] == 0.0  # mtp_engine.py self-test
    parent, mask = O.draft_tree(16, 4, "tree")
    # 64 nodes: 1 + 4 + 16 + 43 (the last level truncated by the node budget)
    depth = [0] * 64
    for n in range(1, 64):
        depth[n] = depth[int(parent[n])] + 1
    assert [depth.count(d) for d in range(4)] == [1, 4, 16, 43]
    for n in range(64):
        anc = {n}
        p = int(parent[n])
        while p >= 0:
            anc.add(p)
            p = int(parent[p])
        assert set(torch.nonzero(mask[n]).flatten().tolist()) == anc


def test_engine_rollback_known_answer():
    draft = torch.tensor([[11, 12, 13, 14], [21, 22, 23, 24]])
    accept = torch.tensor([[1, 1, 0, 0], [1, 1, 1, 1]], dtype=torch.int8)
    n = torch.tensor([2, 4], dtype=torch.int32)
    corr = torch.tensor([5, 6], dtype=torch.int32)
    a_n, rej, toks, adv = O.engine_rollback(accept, n, corr, draft)
    assert (a_n, rej, adv) == (2, True, 3)
    assert toks.tolist() == [[11, 12, 5], [21, 22, 6]]
    a_n, rej, toks, adv = O.engine_rollback(torch.ones(2, 4, dtype=torch.int8),
                                            torch.tensor([4, 4]), corr, draft)
    assert (a_n, rej, adv) == (4, False, 4) and torch.equal(toks, draft)


# --------------------------------------------------------------------------- #
# Attention pins
# --------------------------------------------------------------------------- #
def _attn_brute(q, k, v, valid, scale):
    """float64 loops: softmax over valid keys of q.k*scale, then sum p*v."""
    q, k, v = q.double(), k.double(), v.double()
    L = k.shape[0]
    s = [float((q * k[l]).sum()) * scale for l in range(L)]
    idx = [l for l in range(L) if valid[l]]
    m = max(s[l] for l in idx)
    w = {l: math.exp(s[l] - m) for l in idx}
    z = sum(w.values())
    return sum((w[l] / z) * v[l] for l in idx)


def test_tree_attention_brute_force():
    g = torch.Generator().manual_seed(5)
    B, H, L, D = 2, 3, 11, 8
    q, k, v = (torch.randn(B, H, D, generator=g), torch.randn(B, H, L, D, generator=g),
               torch.randn(B, H, L, D, generator=g))
    mask = (torch.rand(L, generator=g) > 0.4).float()
    mask[3] = 1.0
    out = O.tree_attention(q, k, v, mask)
    for b in range(B):
        for h in range(H):
            ref = _attn_brute(q[b, h], k[b, h], v[b, h], [bool(x > 0.5) for x in mask], 1 / math.sqrt(D))
            assert torch.allclose(out[b, h].double(), ref, atol=1e-5)


def test_tree_attention_all_ones_is_softmax_attention_and_masked_row_is_nan():
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(1, 2, 16, generator=g), torch.randn(1, 2, 9, 16, generator=g),
               torch.randn(1, 2, 9, 16, generator=g))
    out = O.tree_attention(q, k, v, torch.ones(9))
    p = torch.softmax(torch.einsum("bhd,bhld->bhl", q.double(), k.double()) / 4.0, -1)
    ref = torch.einsum("bhl,bhld->bhd", p, v.double())
    assert torch.allclose(out.double(), ref, atol=1e-6)
    assert torch.isnan(O.tree_attention(q, k, v, torch.zeros(9))).all()


def _pages_from_contiguous(k, ps, perm):
    """Pages [P, B, H, ps, D] holding contiguous k [B, H, L, D] with logical page j
    stored at physical page perm[j]; table[b, t] = perm[t // ps]."""
    B, H, L, D = k.shape
    P = len(perm)
    pages = torch.zeros(P, B, H, ps, D, dtype=k.dtype)
    for j in range(L // ps):
        pages[perm[j]] = k[:, :, j * ps:(j + 1) * ps].clone()
    table = torch.tensor([[perm[t // ps] for t in range(L)] for _ in range(B)], dtype=torch.int32)
    return pages, table


def test_paged_attention_equals_contiguous_under_any_page_placement():
    g = torch.Generator().manual_seed(7)
    B, H, L, D, ps = 2, 3, 24, 16, 4
    q = torch.randn(B, H, D, generator=g)
    k = torch.randn(B, H, L, D, generator=g)
    v = torch.randn(B, H, L, D, generator=g)
    ref = O.tree_attention(q, k, v, torch.ones(L))
    for perm in (list(range(L // ps)), [5, 0, 3, 1, 4, 2]):
        kp, table = _pages_from_contiguous(k, ps, perm)
        vp, _ = _pages_from_contiguous(v, ps, perm)
        assert torch.allclose(O.paged_attention(q, kp, vp, table, ps), ref, atol=1e-6)


def test_tree_verify_equals_per_node_single_query_calls():
    g = torch.Generator().manual_seed(8)
    N, H, D, Lc, ps = 5, 2, 16, 12, 4
    _, tm = O.draft_tree(3, 2)
    tm = tm[:N, :N]
    qn = torch.randn(N, H, D, generator=g)
    kc = torch.randn(1, H, Lc, D, generator=g)
    vc = torch.randn(1, H, Lc, D, generator=g)
    kt = torch.randn(N, H, D, generator=g)
    vt = torch.randn(N, H, D, generator=g)
    kp, table = _pages_from_contiguous(kc, ps, [2, 0, 1])
    vp, _ = _pages_from_contiguous(vc, ps, [2, 0, 1])
    out = O.tree_verify_attention(qn, kp, vp, table, ps, kt, vt, tm)
    for n in range(N):
        keys = torch.cat([kc, kt.permute(1, 0, 2)[None]], 2)
        vals = torch.cat([vc, vt.permute(1, 0, 2)[None]], 2)
        mask = torch.cat([torch.ones(Lc), tm[n]])
        ref = O.tree_attention(qn[n][None], keys, vals, mask)[0]
        assert torch.allclose(out[n], ref, atol=1e-6)


def test_verify_tree_mask_pairs():
    """The 64-node tree (depth 16, 4 branches): 1 + 4 + 16 + 43 nodes and
    229 (node, ancestor-or-self) pairs."""
    parent, mask = O.draft_tree(16, 4)
    assert int((parent >= 0).sum()) + 1 == 64
    assert int(mask.sum()) == 229
