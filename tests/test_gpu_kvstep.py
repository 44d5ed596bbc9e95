"""GPU parity of the KV step after verify against the CPU oracle, all
integer / byte work and therefore bit-exact: the batched paged-KV write,
the device-side rollback / commit of the verify outputs (with the id
buffer kept on the device across steps) and the batch prefix match."""
import pytest
import torch

from oracle import eager as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pages(g, B, H, D, P, ps, L, dtype):
    kp = torch.randn(P, B, H, ps, D, generator=g).to(dtype)
    vp = torch.randn(P, B, H, ps, D, generator=g).to(dtype)
    perm = torch.randperm(P, generator=g)
    table = perm[: L // ps].repeat_interleave(ps).reshape(1, L).repeat(B, 1).to(torch.int32)
    return kp, vp, table


@pytest.mark.parametrize("start_kind", ["host", "scalar", "per_row"])
@pytest.mark.parametrize("src,dst", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                     (torch.float32, torch.float32), (torch.float16, torch.float16)])
def test_paged_kv_write_matches_oracle(start_kind, src, dst):
    from mtp_hip import ops
    g = torch.Generator().manual_seed(5)
    B, H, T, D, P, ps, L = 2, 4, 5, 128, 12, 16, 160
    kp, vp, table = _pages(g, B, H, D, P, ps, L, dst)
    table[1, 150:] = -1  # unmapped tail: skipped
    kn = torch.randn(B, H, T, D, generator=g).to(src)
    vn = torch.randn(B, H, T, D, generator=g).to(src)
    if start_kind == "host":
        start, start_dev = 147, 147
    elif start_kind == "scalar":
        start, start_dev = torch.tensor([147]), torch.tensor([147]).to(DEV)
    else:
        start, start_dev = torch.tensor([3, 147]), torch.tensor([3, 147]).to(DEV)
    kd, vd = kp.to(DEV), vp.to(DEV)
    print(f"case kv-write start={start_kind} {src}->{dst}", flush=True)
    ops.paged_kv_write(kn.to(DEV), vn.to(DEV), kd, vd, table.to(DEV), start_dev)
    torch.cuda.synchronize()
    rk, rv = O.paged_kv_write(kn, vn, kp, vp, table, start)
    assert torch.equal(kd.cpu(), rk) and torch.equal(vd.cpu(), rv)


def test_paged_kv_write_then_attention_reads_the_new_keys():
    """Written rows are what the paged attention kernel then reads: the
    attention over the updated cache equals the oracle's on the same cache."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(6)
    B, H, T, D, P, ps, L = 1, 8, 4, 128, 10, 16, 160
    kp, vp, table = _pages(g, B, H, D, P, ps, L, torch.bfloat16)
    kn = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    vn = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    kd, vd, td = kp.to(DEV), vp.to(DEV), table.to(DEV)
    ops.paged_kv_write(kn.to(DEV), vn.to(DEV), kd, vd, td, 100)
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    out = ops.paged_attention(q.to(DEV), kd, vd, td[:, :104].contiguous(), ps)
    torch.cuda.synchronize()
    rk, rv = O.paged_kv_write(kn, vn, kp, vp, table, 100)
    ref = O.paged_attention(q, rk, rv, table[:, :104], ps)
    from conftest import close
    ok, worst = close(out, ref, 2e-2)
    assert ok, worst


def _chain(g, B, D, V):
    top = torch.randint(0, V, (B, D + 1), generator=g)
    from mtp_hip import workloads
    draft = workloads.make_chain_drafts(top, V, int(torch.randint(0, 1000, (1,), generator=g)))
    accept, accepted_n, corrected = O.chain_accept(top, draft)
    return draft, accept, accepted_n, corrected


@pytest.mark.parametrize("B,D", [(8, 4), (1, 1), (3, 0), (64, 7)])
@pytest.mark.parametrize("draft_dtype", [torch.int64, torch.int32])
def test_verify_commit_matches_oracle(B, D, draft_dtype):
    from mtp_hip import ops
    g = torch.Generator().manual_seed(B * 10 + D)
    for trial in range(6):
        draft, acc, n, corr = _chain(g, B, D, 1000)
        if trial == 0 and D > 0:  # full acceptance
            acc = torch.ones(B, D, dtype=torch.int8)
            n = torch.full((B,), D, dtype=torch.int32)
        ck = int(torch.randint(0, 500, (1,), generator=g))
        ckd = torch.tensor([ck], dtype=torch.int64, device=DEV)
        kv = torch.zeros(1, dtype=torch.int64, device=DEV)
        print(f"case commit B={B} D={D} trial={trial}", flush=True)
        tok, width = ops.verify_commit(acc.to(DEV), n.to(DEV), corr.to(DEV),
                                       draft.to(draft_dtype).to(DEV), ckd, kv)
        torch.cuda.synchronize()
        rt, rw, rkv = O.verify_commit(acc, n, corr, draft, ck)
        assert torch.equal(tok.cpu(), rt), (tok.cpu(), rt)
        assert int(width.cpu()) == rw and int(kv.cpu()) == rkv


def test_verify_commit_device_loop_appends_ids_and_aliases_length():
    """Five decode steps without a host read: the KV length scalar is both
    checkpoint and result (aliased), the ids buffer grows on the device; at
    the end it equals the oracle's step-by-step concatenation."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(77)
    B, D, V, prompt = 4, 4, 500, 6
    ids0 = torch.randint(0, V, (B, prompt), generator=g)
    cap = prompt + 5 * (D + 1)
    ids = torch.full((B, cap), -7, dtype=torch.int64)
    ids[:, :prompt] = ids0
    ids_d = ids.to(DEV)
    ids_len = torch.tensor([prompt], dtype=torch.int64, device=DEV)
    kv = torch.tensor([prompt], dtype=torch.int64, device=DEV)
    ref_ids = [ids0]
    ref_kv = prompt
    for step in range(5):
        draft, acc, n, corr = _chain(g, B, D, V)
        ops.verify_commit(acc.to(DEV), n.to(DEV), corr.to(DEV), draft.to(DEV), kv, kv,
                          ids_d, ids_len)
        rt, rw, ref_kv = O.verify_commit(acc, n, corr, draft, ref_kv)
        ref_ids.append(rt[:, :rw])
    torch.cuda.synchronize()
    ref = torch.cat(ref_ids, dim=1)
    assert int(ids_len.cpu()) == ref.shape[1] and int(kv.cpu()) == ref_kv
    assert torch.equal(ids_d.cpu()[:, :ref.shape[1]], ref)
    assert bool((ids_d.cpu()[:, ref.shape[1]:] == -7).all())


@pytest.mark.parametrize("room", [0, 1, 3])
def test_verify_commit_full_id_buffer_stops_at_capacity(room):
    """An id buffer with fewer free columns than the step's width: the
    tokens that fit are written, nothing past the capacity, and ids_len
    stops at the capacity (an advance shorter than width) while the KV
    length still advances by the full width."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(78 + room)
    B, D, V = 3, 4, 300
    draft = torch.randint(0, V, (B, D), generator=g)
    acc = torch.ones(B, D, dtype=torch.int8)  # all accepted: width D
    n = torch.full((B,), D, dtype=torch.int32)
    corr = torch.randint(0, V, (B,), generator=g).to(torch.int32)
    cap, used = 10, 10 - room
    store = torch.full((B * cap + 16,), -9, dtype=torch.int64, device=DEV)
    ids = store[:B * cap].view(B, cap)  # a write past row b's capacity lands in row b + 1
    ids_len = torch.tensor([used], dtype=torch.int64, device=DEV)
    kv = torch.tensor([used], dtype=torch.int64, device=DEV)
    tokens, width = ops.verify_commit(acc.to(DEV), n.to(DEV), corr.to(DEV), draft.to(DEV),
                                      kv, kv, ids, ids_len)
    torch.cuda.synchronize()
    rt, rw, rkv = O.verify_commit(acc, n, corr, draft, used)
    assert int(width.cpu()) == rw == D and int(kv.cpu()) == rkv
    assert int(ids_len.cpu()) == cap
    got = ids.cpu()
    assert torch.equal(got[:, used:], rt[:, :room])
    assert bool((got[:, :used] == -9).all())
    assert bool((store.cpu()[B * cap:] == -9).all())


@pytest.mark.parametrize("R,L", [(1, 5), (2, 0), (7, 5), (5, 64), (9, 65), (300, 1000),
                                 (4097, 33)])
def test_batch_prefix_match_matches_oracle(R, L):
    from mtp_hip import ops
    g = torch.Generator().manual_seed(R + L)
    base = torch.randint(0, 50, (1, L), generator=g)
    ids = base.repeat(R, 1)
    # each row diverges at a random column (or never)
    cut = torch.randint(0, L + 1, (R,), generator=g) if L else torch.zeros(R, dtype=torch.long)
    for r in range(1, R):
        c = int(cut[r])
        if c < L:
            ids[r, c] = (ids[r, c] + 1 + r % 7) % 50
            ids[r, c + 1:] = torch.randint(0, 50, (L - c - 1,), generator=g)
    print(f"case prefix R={R} L={L}", flush=True)
    out = ops.batch_prefix_match(ids.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), O.batch_prefix_match(ids))
