"""Independent pins of the oracle functions that the first set of checks
(test_oracle.py) left open, and of the oracle's draft-chain, decode
attention, monolith and KV-step functions: closed forms, the format
definition of e4m3fn (ties to even), float64 brute force, exhaustive
enumeration and known answers. None of them restates the oracle's formula."""
import math

import numpy as np
import pytest
import torch

from oracle import eager as O

FP8_TABLE = O.fp8_e4m3fn_decode_table()


def _finite_pos_codes():
    """Positive finite e4m3fn codes in increasing value order."""
    codes = [c for c in range(0x00, 0x7F)]  # 0x7f is NaN
    vals = [FP8_TABLE[c] for c in codes]
    assert all(np.diff(vals) > 0)
    return codes, vals


# ---------------------------------------------------------------------------
# quantize_fp8_per_tensor (mtp_kernels.py:704-713)
def test_fp8_per_tensor_scale_closed_form():
    g = torch.Generator().manual_seed(11)
    x = 3.7 * torch.randn(64, 33, generator=g)
    q, s = O.quantize_fp8_per_tensor(x)
    amax = float(np.abs(x.numpy().astype(np.float64)).max())
    # fp32 division amax / 448, as the reference's tensor arithmetic rounds it
    assert float(s) == float(np.float32(np.float32(amax) / np.float32(448.0)))
    assert q.dtype == torch.float8_e4m3fn and q.shape == x.shape
    # all-zero tensor: scale 1, codes 0
    q0, s0 = O.quantize_fp8_per_tensor(torch.zeros(5, 7))
    assert float(s0) == 1.0 and int(q0.view(torch.uint8).max()) == 0


def test_fp8_per_tensor_values_within_half_spacing_and_clamped():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(4096, generator=g) * 10
    q, s = O.quantize_fp8_per_tensor(x)
    codes = q.view(torch.uint8).numpy()
    dec = FP8_TABLE[codes]
    target = np.clip(x.numpy().astype(np.float64) / float(s), -448, 448)
    # spacing around each decoded value from the format table
    _, vals = _finite_pos_codes()
    vals = np.array(vals)
    a = np.abs(dec)
    idx = np.searchsorted(vals, a)
    up = vals[np.minimum(idx + 1, len(vals) - 1)] - a
    down = a - vals[np.maximum(idx - 1, 0)]
    spacing = np.maximum(up, down)
    assert np.all(np.abs(dec - target) <= spacing / 2 + 1e-12)
    assert np.abs(dec).max() <= 448


def test_fp8_per_tensor_ties_go_to_even_code():
    """Every midpoint between adjacent positive e4m3fn values (and their
    negatives) must quantize to the code with the even mantissa bit. 448 in
    the tensor pins the scale at exactly 1."""
    codes, vals = _finite_pos_codes()
    mids, want = [], []
    for (c0, v0), (c1, v1) in zip(zip(codes, vals), zip(codes[1:], vals[1:])):
        mids.append((v0 + v1) / 2)
        want.append(c0 if c0 % 2 == 0 else c1)
        assert (c0 % 2) != (c1 % 2)
    m = np.array(mids, dtype=np.float64)
    assert np.all(m.astype(np.float32).astype(np.float64) == m)  # exact in fp32
    x = torch.tensor(np.concatenate([[448.0], m, -m]), dtype=torch.float32)
    q, s = O.quantize_fp8_per_tensor(x)
    assert float(s) == 1.0
    got = q.view(torch.uint8).numpy()[1:]
    n = len(mids)
    assert np.array_equal(got[:n], np.array(want, dtype=np.uint8))
    assert np.array_equal(got[n:], np.array(want, dtype=np.uint8) | 0x80)


# ---------------------------------------------------------------------------
# dequantize_fp8 (mtp_kernels.py:726-727)
def test_dequantize_fp8_is_table_times_scale():
    allc = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn)
    for s in (1.0, 0.0123, 7.5):
        out = O.dequantize_fp8(allc, torch.tensor(s)).numpy().astype(np.float64)
        ref = FP8_TABLE * np.float64(np.float32(s))
        finite = ~np.isnan(ref)
        # the table value is exact in fp32; one fp32 rounding of the product
        assert np.allclose(out[finite], ref[finite], rtol=2 ** -24, atol=0)
        assert np.all(np.isnan(out[~finite]))
    # per-row scales broadcast over the row
    q = allc[:252].reshape(4, 63)
    sc = torch.tensor([[0.5], [2.0], [1.0], [0.25]])
    out = O.dequantize_fp8(q, sc).numpy()
    ref = FP8_TABLE[:252].reshape(4, 63) * sc.numpy().astype(np.float64)
    assert np.array_equal(out[~np.isnan(ref)], ref[~np.isnan(ref)].astype(np.float32))


# ---------------------------------------------------------------------------
# pack_scales / unpack_scale_tensor (mtp_kernels.py:1336-1353), oracle and product
@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_pack_scales_offsets_and_roundtrip(impl):
    if impl == "oracle":
        pack = O.pack_scales
        from mtp_hip.kernels import unpack_scale_tensor as unpack
    else:
        from mtp_hip.kernels import pack_scales as pack, unpack_scale_tensor as unpack
    g = torch.Generator().manual_seed(5)
    ws = [torch.rand(7, generator=g), torch.rand(3, 4, generator=g).half()]
    kv = [torch.rand(2, generator=g), torch.rand(5, generator=g).double()]
    flat, offs = pack(ws, kv)
    sizes = [7, 12, 2, 5]
    assert offs.dtype == torch.int64
    assert offs.tolist() == [0, 7, 19, 21, 26]  # closed form: running sums
    assert flat.dtype == torch.float32 and flat.numel() == sum(sizes)
    for i, t in enumerate(ws + kv):
        back = unpack(flat, offs, i, tuple(t.shape))
        assert back.shape == t.shape
        assert torch.equal(back, t.float())
    flat2, offs2 = pack(ws)
    assert offs2.tolist() == [0, 7, 19] and flat2.numel() == 19


# ---------------------------------------------------------------------------
# rmsnorm / add_rmsnorm (mtp_kernels.py:910-933, 1082-1102)
def brute_rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    out = np.empty_like(x)
    for m in range(x.shape[0]):
        rs = 1.0 / math.sqrt(sum(v * v for v in x[m]) / x.shape[1] + eps)
        out[m] = [x[m, i] * rs * w[i] for i in range(x.shape[1])]
    return out


def test_rmsnorm_reference_check_and_brute_force():
    # the reference's own check (test_engine.py:4): seed 0, [7, 32], < 1e-4
    torch.manual_seed(0)
    A = torch.randn(7, 32)
    Bw = torch.randn(32)
    y = O.rmsnorm(A, Bw, 1e-6)
    ref = brute_rmsnorm(A.numpy(), Bw.numpy().astype(np.float64), 1e-6)
    assert np.abs(y.numpy() - ref).max() < 1e-4
    assert np.abs(y.numpy() - ref).max() < 1e-5 * np.abs(ref).max()


def test_rmsnorm_constant_row_closed_form_and_weight_cast():
    c, eps = 3.0, 1e-6
    x = torch.full((2, 16), c)
    y = O.rmsnorm(x, None, eps)
    assert np.allclose(y.numpy(), c / math.sqrt(c * c + eps), rtol=1e-7)
    # bf16 x: the weight is rounded to bf16 before use (the wrapper's cast)
    xb = torch.tensor([[1.0, -1.0, 1.0, -1.0]], dtype=torch.bfloat16)
    w = torch.tensor([1.00390625 + 2 ** -10] * 4)  # not a bf16 value
    yb = O.rmsnorm(xb, w, 0.0)
    wb = float(w[0].to(torch.bfloat16))
    assert yb.dtype == torch.bfloat16
    assert float(yb[0, 0]) == float(torch.tensor(wb).to(torch.bfloat16))


def test_add_rmsnorm_is_rmsnorm_of_fp32_sum():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(5, 40, generator=g)
    r = torch.randn(5, 40, generator=g)
    w = torch.randn(40, generator=g)
    y = O.add_rmsnorm(x, r, w, 1e-6)
    ref = brute_rmsnorm((x.double() + r.double()).numpy(), w.double().numpy(), 1e-6)
    assert np.abs(y.numpy() - ref).max() < 1e-5 * np.abs(ref).max()


# ---------------------------------------------------------------------------
# argmax_tokens (mtp_perf_hardening.py:170-186)
def test_argmax_tokens_brute_force_ties_nan_and_gather():
    g = torch.Generator().manual_seed(4)
    lg = torch.randint(-3, 4, (6, 50), generator=g).float()
    lg[2, 7] = float("nan")
    lg[2, 30] = float("nan")
    lg[4] = -math.inf
    tab = torch.randn(50, 3, generator=g)
    tok, emb = O.argmax_tokens(lg, tab)
    for m in range(6):
        row = lg[m].tolist()
        if any(v != v for v in row):
            want = next(i for i, v in enumerate(row) if v != v)
        else:
            best = max(row)
            want = next(i for i, v in enumerate(row) if v == best)
        assert int(tok[m]) == want
        assert torch.equal(emb[m], tab[want])
    assert tok.dtype == torch.int64


# ---------------------------------------------------------------------------
# causal attention, fp8 KV (mtp_kernels.py:980-1011, 1105-1133)
def brute_attend(q, K, V, scale):
    s = [sum(q[d] * K[l][d] for d in range(len(q))) * scale for l in range(len(K))]
    m = max(s)
    p = [math.exp(v - m) for v in s]
    tot = sum(p)
    return [sum(p[l] * V[l][d] for l in range(len(K))) / tot for d in range(len(q))]


def test_causal_attention_brute_force():
    g = torch.Generator().manual_seed(21)
    q = torch.randn(2, 3, 8, generator=g)
    k = torch.randn(2, 3, 11, 8, generator=g)
    v = torch.randn(2, 3, 11, 8, generator=g)
    out = O.causal_attention(q, k, v)
    for b in range(2):
        for h in range(3):
            ref = brute_attend(q[b, h].double().tolist(), k[b, h].double().tolist(),
                               v[b, h].double().tolist(), 1 / math.sqrt(8))
            assert np.allclose(out[b, h].numpy(), ref, rtol=1e-5, atol=1e-6)


def test_causal_attention_fp8_dequantises_per_head():
    g = torch.Generator().manual_seed(22)
    q = torch.randn(1, 2, 8, generator=g)
    k8 = (torch.randn(1, 2, 9, 8, generator=g) * 50).to(torch.float8_e4m3fn)
    v8 = (torch.randn(1, 2, 9, 8, generator=g) * 50).to(torch.float8_e4m3fn)
    ks, vs = torch.tensor([0.01, 0.02]), torch.tensor([0.5, 0.03])
    out = O.causal_attention_fp8(q, k8, v8, ks, vs)
    for h in range(2):
        K = FP8_TABLE[k8[0, h].view(torch.uint8).numpy()] * float(ks[h])
        V = FP8_TABLE[v8[0, h].view(torch.uint8).numpy()] * float(vs[h])
        ref = brute_attend(q[0, h].double().tolist(), K.tolist(), V.tolist(), 1 / math.sqrt(8))
        assert np.allclose(out[0, h].numpy(), ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# tree monolith (mtp_kernels.py:881-907, 1222-1250)
def test_tree_attn_rmsnorm_linear_brute_force_and_all_masked_nan():
    g = torch.Generator().manual_seed(23)
    B, H, D, L, N = 2, 2, 8, 6, 5
    q = torch.randn(B, H, D, generator=g)
    k = torch.randn(B, H, L, D, generator=g)
    v = torch.randn(B, H, L, D, generator=g)
    mask = torch.tensor([1.0, 0.0, 1.0, 1.0, 0.2, 0.9])
    W = torch.randn(N, D, generator=g)
    gam = 1 + 0.1 * torch.randn(D, generator=g)
    bias = torch.randn(N, generator=g)
    wsc = torch.rand(N, generator=g) + 0.5
    out = O.tree_attn_rmsnorm_linear(q, k, v, mask, W, gam, bias, wsc, None, 1e-6)
    keep = [i for i in range(L) if mask[i] > 0.5]
    for b in range(B):
        for h in range(H):
            a = brute_attend(q[b, h].double().tolist(), k[b, h, keep].double().tolist(),
                             v[b, h, keep].double().tolist(), 1 / math.sqrt(D))
            rs = 1 / math.sqrt(sum(t * t for t in a) / D + 1e-6)
            an = [a[d] * rs * float(gam[d]) for d in range(D)]
            ref = [sum(an[d] * float(W[n, d]) * float(wsc[n]) for d in range(D)) + float(bias[n])
                   for n in range(N)]
            assert np.allclose(out[b, h].numpy(), ref, rtol=1e-5, atol=1e-5)
    nan = O.tree_attn_rmsnorm_linear(q, k, v, torch.zeros(L), W)
    assert bool(torch.isnan(nan).all())


# ---------------------------------------------------------------------------
# KV step (mtp_engine.py:581-585, 1244-1258; mtp_radix.py:195-236)
def test_paged_kv_write_elementwise_and_readback():
    g = torch.Generator().manual_seed(31)
    B, H, T, D, P, ps, L = 2, 3, 5, 4, 6, 4, 16
    kp = torch.zeros(P, B, H, ps, D)
    vp = torch.zeros(P, B, H, ps, D)
    table = torch.randperm(P, generator=g)[:L // ps].repeat_interleave(ps).reshape(1, L).repeat(B, 1)
    table = table.to(torch.int32)
    table[1, 12:] = -1  # unmapped: skipped
    kn = torch.randn(B, H, T, D, generator=g)
    vn = torch.randn(B, H, T, D, generator=g)
    start = 9
    k2, v2 = O.paged_kv_write(kn, vn, kp, vp, table, start)
    for b in range(B):
        for h in range(H):
            for t in range(T):
                p = start + t
                pid = int(table[b, p])
                if pid < 0:
                    continue
                assert torch.equal(k2[pid, b, h, p % ps], kn[b, h, t])
                assert torch.equal(v2[pid, b, h, p % ps], vn[b, h, t])
    written = sum(1 for b in range(B) for t in range(T) if int(table[b, start + t]) >= 0)
    assert int((k2 != 0).any(-1).sum()) == written * H
    # read back through the paged attention oracle: keys 9..13 of row 0
    q = torch.randn(B, H, D, generator=g)
    tab0 = table[:, 9:12].contiguous()
    k_rows = torch.stack([k2[tab0[b, i], b, :, (9 + i) % ps] for b in range(B) for i in range(3)])
    assert torch.equal(k_rows.reshape(B, 3, H, D).permute(0, 2, 1, 3), kn[:, :, :3])


def test_verify_commit_known_answers():
    draft = torch.tensor([[5, 6, 7], [8, 9, 10]])
    # full acceptance: the whole draft, width D
    acc = torch.ones(2, 3, dtype=torch.int8)
    tok, w, kv = O.verify_commit(acc, torch.tensor([3, 3]), torch.tensor([1, 2]), draft, 100)
    assert w == 3 and kv == 103 and tok.tolist() == [[5, 6, 7, -1], [8, 9, 10, -1]]
    # row 1 rejects at d = 1: a_n = min(3, 1) = 1 -> draft[:, :1] ++ corrected
    acc = torch.tensor([[1, 1, 1], [1, 0, 0]], dtype=torch.int8)
    tok, w, kv = O.verify_commit(acc, torch.tensor([3, 1]), torch.tensor([40, 41]), draft, 50)
    assert w == 2 and kv == 52 and tok.tolist() == [[5, 40, -1, -1], [8, 41, -1, -1]]
    # immediate rejection everywhere: only the corrected token
    acc = torch.zeros(2, 3, dtype=torch.int8)
    tok, w, kv = O.verify_commit(acc, torch.tensor([0, 0]), torch.tensor([3, 4]), draft, 7)
    assert w == 1 and kv == 8 and tok.tolist() == [[3, -1, -1, -1], [4, -1, -1, -1]]


def test_batch_prefix_match_brute_force():
    g = torch.Generator().manual_seed(41)
    for R, L in ((1, 5), (2, 0), (5, 9), (7, 70)):
        ids = torch.randint(0, 3, (R, L), generator=g)
        if R > 2 and L:
            ids[2] = ids[0]
        out = O.batch_prefix_match(ids)
        for r in range(R):
            if R <= 1:
                want = 0
            else:
                want = next((c for c in range(L) if ids[r, c] != ids[0, c]), L)
            assert int(out[r]) == want
        assert out.dtype == torch.int32
