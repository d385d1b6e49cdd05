"""Pins the CPU oracle against independent anchors (no GPU needed).

Each oracle function is checked against something other than its own
formula: torch's CPU kernels (argmax, bf16 and float8 casts, bf16 add, cat,
index_select), hand-worked vectors written from the reference source
(tests/golden/accept_cases.json), numpy dense attention with an explicit
mask over pages gathered through the block table, and closed forms (one
visible key, equal scores, round trips).
"""
import json
import os

import numpy as np
import pytest
import torch

from helpers import acceptance_logits, bits, paged_case
from oracle import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- argmax / accept

def test_argmax_matches_torch_on_random_and_special_rows():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(12, 3001, generator=g).to(torch.bfloat16)
    xb = x.view(torch.int16)
    x[0, 10] = 9.0
    x[0, 2000] = 9.0
    xb[1, 7] = 0x7FC1
    xb[1, 3] = -64
    x[2, :] = -1.0
    x[2, 50] = -0.0
    x[2, 60] = 0.0
    x[3, :] = float("-inf")
    x[4, :] = 0.0
    x[5, 3000] = 100.0
    x[6, 0] = float("inf")
    x[6, 1] = float("inf")
    x[7, :] = float("nan")
    np.testing.assert_array_equal(oracle.argmax_bf16(bits(x)), x.argmax(-1).numpy())


def test_argmax_brute_force_all_small_rows():
    # every row over a 4-symbol alphabet including NaN / -0 / +0 / -inf
    symbols = torch.tensor([float("nan"), -0.0, 0.0, float("-inf"), 1.0], dtype=torch.bfloat16)
    idx = torch.cartesian_prod(*[torch.arange(5)] * 4)
    rows = symbols[idx]
    np.testing.assert_array_equal(oracle.argmax_bf16(bits(rows)), rows.argmax(-1).numpy())


def test_accept_hand_worked_vectors():
    cases = json.load(open(os.path.join(GOLDEN, "accept_cases.json")))["cases"]
    for c in cases:
        if "error" in c:
            with pytest.raises(ValueError):
                oracle.verify_greedy_proposals(c["proposal"], c["target"])
            continue
        v = oracle.verify_greedy_proposals(c["proposal"], c["target"])
        assert v.accepted_count == c["accepted"]
        assert v.accepted_tokens == c["tokens"]
        assert v.replacement_token == c["replacement"]
        if len(c["target"]) == len(c["proposal"]) + 1:
            # the batched C restatement on the verify-row layout
            q = len(c["target"])
            ids = np.array([99] + c["proposal"], np.int64)
            acc, bonus = oracle.accept(np.array([0, q], np.int32), np.array(c["target"], np.int32), ids)
            assert acc[0] == c["accepted"] and bonus[0] == c["replacement"]


def test_accept_batch_matches_python_restatement():
    logits, cu_q, ids, prop = acceptance_logits(8, 4, 4096, 0.7, 0)
    am = oracle.argmax_bf16(bits(logits))
    acc, bonus = oracle.accept(cu_q.numpy(), am, ids.numpy())
    for s in range(8):
        target = am[s * 5:(s + 1) * 5].tolist()
        v = oracle.verify_greedy_proposals(prop[s].tolist(), target)
        assert acc[s] == v.accepted_count and bonus[s] == v.replacement_token
    assert acc.max() > 0  # raised draft logits do get accepted
    a2, b2, committed = oracle.reference_cpu_acceptance(logits, cu_q.tolist(), ids.tolist())
    assert a2 == acc.tolist() and b2 == bonus.tolist()
    assert committed == int(acc.sum()) + 8


def test_oracle_on_the_committed_config1_fixture():
    """BASELINE config 1 at a reduced vocabulary, frozen with its expected
    outputs (tests/golden/gen_config1_fixture.py: numpy argmax and a plain
    first-mismatch scan, no oracle code)."""
    f = np.load(os.path.join(GOLDEN, "config1_reduced.npz"))
    am = oracle.argmax_bf16(f["logits_bits"])
    np.testing.assert_array_equal(am, f["argmax"])
    acc, bonus = oracle.accept(f["cu_q"], am, f["input_ids"])
    np.testing.assert_array_equal(acc, f["accept_len"])
    np.testing.assert_array_equal(bonus, f["bonus"])
    assert set(f["accept_len"].tolist()) >= {0, 1, 4}   # none, partial and full acceptance


def test_accept_empty_sequence():
    acc, bonus = oracle.accept(np.array([0, 0, 2], np.int32), np.array([4, 5], np.int32),
                               np.array([1, 4], np.int64))
    assert acc.tolist() == [0, 1] and bonus.tolist() == [-1, 5]


# ---------------------------------------------------------------- conversions

def test_e4m3_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.e4m3_to_f32(codes)
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got))
    np.testing.assert_array_equal(got[~nan], ref[~nan])


def test_e4m3_encode_every_bf16_matches_torch_in_range():
    pat = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = oracle.bf16_bits_to_f32(pat)
    got = oracle.f32_to_e4m3(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    finite_small = np.isfinite(x) & (np.abs(x) < 464.0)
    np.testing.assert_array_equal(got[finite_small], ref[finite_small])
    # NaN keeps its sign; everything else saturates to +-448 (0x7E)
    nan = np.isnan(x)
    assert np.all((got[nan] & 0x7F) == 0x7F)
    big = ~nan & ~finite_small
    assert np.all((got[big] & 0x7F) == 0x7E)
    assert np.all((got[big] >> 7) == (x[big] < 0))


def test_e4m3_encode_ties_round_to_even():
    # midpoints between adjacent codes round to the even code
    for c in range(0, 0x7D):
        a = float(oracle.e4m3_to_f32(np.array([c], np.uint8))[0])
        b = float(oracle.e4m3_to_f32(np.array([c + 1], np.uint8))[0])
        mid = np.float32((a + b) / 2)
        want = c if c % 2 == 0 else c + 1
        assert oracle.f32_to_e4m3(np.array([mid]))[0] == want, c
    x = torch.randn(20000, generator=torch.Generator().manual_seed(1)) * 30
    got = oracle.f32_to_e4m3(x.numpy())
    ref = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, ref)


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(2)
    x = torch.cat([torch.randn(5000, generator=g) * 10.0 ** e for e in (-30, -3, 0, 3, 30)])
    x = torch.cat([x, torch.tensor([float("inf"), float("-inf"), 3.3895314e38, -0.0, 1e-45])])
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits(x.numpy()), bits(x.to(torch.bfloat16)))


# ---------------------------------------------------------------- store / rollback

@pytest.mark.parametrize("fp8", [False, True])
def test_store_kv_round_trip(fp8):
    g = torch.Generator().manual_seed(3)
    t, hkv, d, nb, bs = 40, 2, 16, 3, 32
    key = (torch.randn(t, hkv, d, generator=g) * 0.5).to(torch.bfloat16)
    val = (torch.randn(t, hkv, d, generator=g) * 0.5).to(torch.bfloat16)
    slots = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    slots[3] = -1
    slots[5] = nb * bs + 7        # out of range: skipped
    dt = np.uint8 if fp8 else np.uint16
    kc = np.full((nb, bs, hkv, d), 0x11, dt)
    vc = np.full((nb, bs, hkv, d), 0x11, dt)
    oracle.store_kv(bits(key), bits(val), kc, vc, slots.numpy())
    flat_k = kc.reshape(nb * bs, hkv, d)
    flat_v = vc.reshape(nb * bs, hkv, d)
    for i in range(t):
        s = int(slots[i])
        if s < 0 or s >= nb * bs:
            continue
        if fp8:
            ref_k = key[i].float().to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            ref_v = val[i].float().to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        else:
            ref_k, ref_v = bits(key[i]), bits(val[i])
        np.testing.assert_array_equal(flat_k[s], ref_k)
        np.testing.assert_array_equal(flat_v[s], ref_v)
    written = {int(s) for s in slots if 0 <= int(s) < nb * bs}
    untouched = [s for s in range(nb * bs) if s not in written]
    assert np.all(flat_k[untouched] == 0x11)


def test_rollback_hand_case():
    cu = np.array([0, 5, 6, 9], np.int32)
    acc = np.array([2, 0, -3], np.int32)        # -3 clamps to 0
    slots = np.arange(9, dtype=np.int32) + 100
    lens = np.array([50, 7, 30], np.int32)
    kc = np.ones((1, 256, 1, 4), np.uint16)
    vc = np.ones((1, 256, 1, 4), np.uint16)
    s2, l2 = oracle.rollback(cu, acc, slots, lens, kc, vc, poison=True)
    assert s2.tolist() == [100, 101, 102, -1, -1, 105, 106, -1, -1]
    assert l2.tolist() == [48, 7, 28]
    zeroed = [103, 104, 107, 108]
    assert np.all(kc[0, zeroed] == 0) and np.all(vc[0, zeroed] == 0)
    assert np.all(np.delete(kc[0], zeroed, axis=0) == 1)


# ---------------------------------------------------------------- aux gather

def test_aux_gather_matches_torch():
    g = torch.Generator().manual_seed(4)
    t, h = 30, 64
    hid = [(torch.randn(t, h, generator=g) * 10 ** i).to(torch.bfloat16) for i in range(3)]
    res = [(torch.randn(t, h, generator=g) * 10 ** (2 - i)).to(torch.bfloat16) for i in range(3)]
    hid[0][1, 0] = float("inf")
    res[0][1, 0] = float("-inf")
    src = torch.tensor([4, 0, 29, 4, 17], dtype=torch.int32)
    ref = torch.cat([a + b for a, b in zip(hid, res)], dim=-1).index_select(0, src.long())
    got = oracle.aux_gather([bits(a) for a in hid], [bits(b) for b in res], src.numpy())
    np.testing.assert_array_equal(got, bits(ref))


# ---------------------------------------------------------------- attention

def _dense_reference(case, q_bits=None):
    """numpy dense attention: gather each sequence's pages into a contiguous
    [L, Hkv, D] matrix first, then softmax(QK^T + mask) V with an explicit
    bottom-right causal mask -- a different code path from the oracle."""
    bs = case["block_size"]
    q = case["q"].double().numpy()
    kc = case["k_cache"].double().numpy()
    vc = case["v_cache"].double().numpy()
    hq, hkv = q.shape[1], kc.shape[2]
    out = np.zeros(q.shape)
    for i, (L, qn) in enumerate(zip(case["lens"].tolist(), case["q_lens"])):
        blocks = case["block_tables"][i, :(L + bs - 1) // bs].long().numpy()
        k = kc[blocks].reshape(-1, hkv, q.shape[2])[:L]
        v = vc[blocks].reshape(-1, hkv, q.shape[2])[:L]
        s0 = int(case["cu_q"][i])
        rows = np.arange(qn)[:, None]
        cols = np.arange(L)[None, :]
        mask = cols <= (L - qn + rows)
        for h in range(hq):
            sc = q[s0:s0 + qn, h] @ k[:, h // (hq // hkv)].T * q.shape[2] ** -0.5
            sc = np.where(mask, sc, -np.inf)
            w = np.exp(sc - sc.max(-1, keepdims=True))
            w /= w.sum(-1, keepdims=True)
            out[s0:s0 + qn, h] = w @ v[:, h // (hq // hkv)]
    return out


@pytest.mark.parametrize("kw", [
    dict(seed=1, batch=3, q_len=5, ctx_lo=5, ctx_hi=600, hq=4, hkv=2, head_dim=32, block_size=64),
    dict(seed=2, batch=4, q_len=[1, 2, 7, 3], ctx_lo=1, ctx_hi=300, hq=8, hkv=1, head_dim=16,
         block_size=32),
])
def test_paged_attention_matches_dense_numpy(kw):
    case = paged_case(**kw)
    got = oracle.paged_attention(bits(case["q"]), bits(case["k_cache"]), bits(case["v_cache"]),
                                 case["cu_q"].numpy(), case["lens"].numpy(),
                                 case["block_tables"].numpy(), case["q"].shape[2] ** -0.5)
    ref = _dense_reference(case)
    assert np.abs(got - ref).max() < 1e-6


def test_paged_attention_closed_forms():
    # one visible key -> output equals that value row; equal scores -> mean
    d, bs = 8, 32
    q = torch.zeros(2, 1, d).to(torch.bfloat16)
    q[0, 0, 0] = 1.0
    kc = torch.zeros(2, bs, 1, d)
    vc = torch.arange(2 * bs * d, dtype=torch.float32).reshape(2, bs, 1, d) / 64
    bt = np.array([[1, 0]], np.int32)
    # sequence of 3 keys, 2 query rows: row 0 sees keys 0..1, row 1 sees 0..2
    out = oracle.paged_attention(bits(q), bits(kc.to(torch.bfloat16)), bits(vc.to(torch.bfloat16)),
                                 np.array([0, 2], np.int32), np.array([3], np.int32), bt, 1.0)
    vb = vc.to(torch.bfloat16).float().numpy()
    np.testing.assert_allclose(out[0, 0], vb[1, 0:2, 0].mean(0), rtol=1e-6)
    np.testing.assert_allclose(out[1, 0], vb[1, 0:3, 0].mean(0), rtol=1e-6)
    # L=1, q=1 -> exactly the single value row
    out1 = oracle.paged_attention(bits(q[:1]), bits(kc.to(torch.bfloat16)),
                                  bits(vc.to(torch.bfloat16)), np.array([0, 1], np.int32),
                                  np.array([1], np.int32), bt, 1.0)
    np.testing.assert_array_equal(out1[0, 0], vb[1, 0, 0])


def test_fp8_decode_restatement_within_reference_bound():
    torch.manual_seed(0)
    length, bs, hkv, hq, d = 300, 256, 2, 4, 128
    key = (torch.randn(length, hkv, d) * 0.1).to(torch.bfloat16)
    val = (torch.randn(length, hkv, d) * 0.1).to(torch.bfloat16)
    kc = np.zeros((2, bs, hkv, d), np.uint8)
    vc = np.zeros((2, bs, hkv, d), np.uint8)
    table = np.array([[1, 0]], np.int32)
    pos = np.arange(length)
    slots = (table[0, pos // bs] * bs + pos % bs).astype(np.int32)
    oracle.store_kv(bits(key), bits(val), kc, vc, slots)
    q = (torch.randn(1, hq, d) * 0.1).to(torch.bfloat16)
    for n in (1, 113, 300):
        got = oracle.fp8_paged_decode(bits(q), kc, vc, np.array([n], np.int32), table, d ** -0.5)
        ref = oracle.paged_attention(bits(q), kc, vc, np.array([0, 1], np.int32),
                                     np.array([n], np.int32), table, d ** -0.5)
        assert np.abs(got - ref).max() <= 2e-3


# ---------------------------------------------------------------- verify metadata

def test_verify_metadata_reference_decode_vector():
    """tests/test_decode_context.py:26-32 of the reference: one row per
    sequence at its last position."""
    cu_q, cu_k, pos, slots = oracle.verify_metadata([15, 16], [1, 1], [[3], [5]], 256, 2)
    assert pos.tolist() == [15, 16]
    assert slots.tolist() == [3 * 256 + 15, 5 * 256 + 16]
    assert cu_q.tolist() == [0, 1, 2] and cu_k.tolist() == [0, 16, 33]


def test_verify_metadata_hand_worked_page_crossing():
    # rows at positions 254..259 cross from logical block 0 (physical 7) into
    # logical block 1 (physical 2); a padded -1 entry and padding rows follow
    cu_q, cu_k, pos, slots = oracle.verify_metadata([254, 0], [6, 2], [[7, 2, -1], [-1, -1, -1]],
                                                   256, 10)
    assert pos.tolist() == [254, 255, 256, 257, 258, 259, 0, 1, 0, 0]
    assert slots.tolist() == [7 * 256 + 254, 7 * 256 + 255, 512, 513, 514, 515, -1, -1, -1, -1]
    assert cu_q.tolist() == [0, 6, 8] and cu_k.tolist() == [0, 260, 262]


def test_verify_metadata_agrees_with_engine_host_path(monkeypatch):
    """The engine's host-side prepare_prefill (the eager path, written
    independently of the restatement) gives the same positions, slots and
    offsets for verify windows."""
    import random

    import torch

    from nanovllm_amd.context import get_context, reset_context
    from nanovllm_amd.engine import model_runner as mr
    from nanovllm_amd.engine.sequence import Sequence

    monkeypatch.setattr(mr, "_pinned", lambda values, dtype: torch.tensor(values, dtype=dtype))
    rng = random.Random(5)
    runner = mr.ModelRunner.__new__(mr.ModelRunner)
    runner.block_size = 256
    runner.device = torch.device("cpu")
    seqs, starts, qs, tables = [], [], [], []
    for _ in range(7):
        n = rng.randrange(1, 900)
        seq = Sequence(list(range(n)))
        seq.block_table = rng.sample(range(100), -(-n // 256))
        q = rng.randrange(1, 7)
        seq.num_computed_tokens = n - q
        seq.num_scheduled_tokens = q
        seqs.append(seq)
        starts.append(n - q)
        qs.append(q)
        tables.append(seq.block_table + [-1] * (4 - len(seq.block_table)))
    try:
        _, pos = runner.prepare_prefill(seqs)
        ctx = get_context()
        ocu_q, ocu_k, opos, oslots = oracle.verify_metadata(starts, qs, tables, 256, pos.numel())
        assert opos.tolist() == pos.tolist()
        assert oslots.tolist() == ctx.slot_mapping.tolist()
        assert ocu_q.tolist() == ctx.cu_seqlens_q.tolist()
        assert ocu_k.tolist() == ctx.cu_seqlens_k.tolist()
    finally:
        reset_context()


def test_commit_metadata_hand_worked():
    # two sequences of a q = 3 verify batch accept 1 and 2 drafts: sequence 0
    # commits verify rows 0, 1 at positions 10, 11 (physical block 7);
    # sequence 1 commits rows 3, 4, 5 at positions 255 .. 257, crossing from
    # physical block 4 into physical block 9; one padding row follows
    am = [100, 101, 102, 103, 104, 105]
    cu_q, cu_k, pos, slots, rows, ids, last = oracle.commit_metadata(
        [10, 255], [1, 2], 3, am, [[7, 8], [4, 9]], 256, 6)
    assert cu_q.tolist() == [0, 2, 5] and cu_k.tolist() == [0, 12, 270]
    assert pos.tolist() == [10, 11, 255, 256, 257, 0]
    assert slots.tolist() == [7 * 256 + 10, 7 * 256 + 11, 4 * 256 + 255, 9 * 256, 9 * 256 + 1, -1]
    assert rows.tolist() == [0, 1, 3, 4, 5, -1]
    assert ids.tolist() == [100, 101, 103, 104, 105, 100]
    assert last.tolist() == [1, 4]
    # accept lengths outside [0, q - 1] are clamped to one and to q rows
    cu_q, _, _, _, rows, _, last = oracle.commit_metadata([0, 0], [-4, 9], 3, am, [[1], [2]],
                                                          256, 6)
    assert cu_q.tolist() == [0, 1, 4] and rows.tolist() == [0, 3, 4, 5, -1, -1]
    assert last.tolist() == [0, 3]


def test_commit_metadata_reference_slot_convention_hand_worked():
    """The reference's commit (_commit_eagle3_tokens, model_runner.py:
    1127-1156) writes tail token i of a commit starting at start_position s
    at slot position s + 1 + i with context s + 2 + i.  Worked by hand for
    s = 254, three tokens, block table [7, 2] (256-token pages): slot
    positions 255, 256, 257 -> slots 7*256+255, 2*256+0, 2*256+1, contexts
    256, 257, 258.  The batched form gives the sequence 258 keys, so its
    bottom-right aligned row j sees 258 - 3 + j + 1 = 256 + j keys, the
    reference's context for token j.  With slot_offset 0 every position
    keeps its own slot (254 -> 7*256+254) and the sequence 257 keys."""
    am = list(range(100, 106))
    cu_q, cu_k, pos, slots, rows, ids, last = oracle.commit_metadata(
        [254], [2], 6, am, [[7, 2]], 256, 4, slot_offset=1)
    assert pos.tolist() == [254, 255, 256, 0]
    assert slots.tolist() == [7 * 256 + 255, 2 * 256 + 0, 2 * 256 + 1, -1]
    assert cu_q.tolist() == [0, 3] and cu_k.tolist() == [0, 258]
    n_keys = int(cu_k[1] - cu_k[0])
    assert [n_keys - 3 + j + 1 for j in range(3)] == [256, 257, 258]
    assert rows.tolist() == [0, 1, 2, -1] and ids.tolist() == [100, 101, 102, 100]
    assert last.tolist() == [2]
    cu_q, cu_k, pos, slots, *_ = oracle.commit_metadata([254], [2], 6, am, [[7, 2]], 256, 4)
    assert pos.tolist() == [254, 255, 256, 0]
    assert slots.tolist() == [7 * 256 + 254, 7 * 256 + 255, 2 * 256 + 0, -1]
    assert cu_k.tolist() == [0, 257]
    # the reference's slot for the last committed token may fall in a page
    # the table does not have: slot -1 (no write) rather than an error
    _, _, _, slots, *_ = oracle.commit_metadata([510], [1], 6, am, [[7, 2]], 256, 2,
                                                slot_offset=1)
    assert slots.tolist() == [2 * 256 + 255, -1]


def test_draft_metadata_reference_slot_convention_hand_worked():
    """_set_eagle3_decode_context (model_runner.py:1087-1096): for a
    sequence of len(seq) tokens, draft step `step` queries RoPE position
    len - 1 + step, writes slot position len + step and sees len + step + 1
    keys.  Worked by hand: length 253 before the verify, one accepted draft
    plus the bonus -> len 255 after it; block table [7, 2, -1]; three
    steps.  Reference (offset 1): slot positions 255, 256, 257 -> slots
    2047, 512, 513, contexts 256, 257, 258.  Offset 0: slot positions 254,
    255, 256 -> 2046, 2047, 512, contexts 255, 256, 257.  The second column
    is padding (position 0, slot -1, context 1); a third sequence's late
    steps run past its one-page table (slot -1)."""
    lens, vrow, accept = [253, 0, 250], [1, 0, 2], [9, 1, 3]
    tables = [[7, 2, -1], [-1, -1, -1], [4, -1, -1]]
    pos, slots, ctx = oracle.draft_metadata(lens, vrow, accept, 1, 2, 3, tables, 256,
                                            slot_offset=1)
    assert pos.tolist() == [[254, 0], [255, 0], [256, 0]]
    assert slots.tolist() == [[2047, -1], [512, -1], [513, -1]]
    assert ctx.tolist() == [[256, 1], [257, 1], [258, 1]]
    pos, slots, ctx = oracle.draft_metadata(lens, vrow, accept, 1, 2, 3, tables, 256)
    assert pos.tolist() == [[254, 0], [255, 0], [256, 0]]
    assert slots.tolist() == [[2046, -1], [2047, -1], [512, -1]]
    assert ctx.tolist() == [[255, 1], [256, 1], [257, 1]]
    # the third sequence: 250 + 3 + 1 = 254 tokens; reference slot
    # positions 254, 255, 256 -> 4*256+254, 4*256+255, past the table
    pos, slots, ctx = oracle.draft_metadata([lens[2]], [0], [3], 1, 1, 3, [tables[2]], 256,
                                            slot_offset=1)
    assert pos[:, 0].tolist() == [253, 254, 255]
    assert slots[:, 0].tolist() == [4 * 256 + 254, 4 * 256 + 255, -1]
    assert ctx[:, 0].tolist() == [255, 256, 257]


def test_draft_metadata_offset_zero_agrees_with_engine_host_loop():
    """Offset 0 is what the engine's own host loop builds for a fresh draft
    (ModelRunner._draft_step_metadata, written independently): the same
    positions, slots and contexts for sequences of the post-verify
    lengths, on random batches."""
    import random

    from nanovllm_amd.engine import model_runner as mr
    from nanovllm_amd.engine.sequence import Sequence

    rng = random.Random(17)
    runner = mr.ModelRunner.__new__(mr.ModelRunner)
    runner.block_size = 256
    for trial in range(10):
        b, k = rng.randrange(1, 9), rng.randrange(2, 8)
        lens = [rng.randrange(1, 1200) for _ in range(b)]
        accept = [rng.randrange(0, k) for _ in range(b)]
        vrow = list(range(b))
        rng.shuffle(vrow)
        acc_by_row = [0] * b
        for i in range(b):
            acc_by_row[vrow[i]] = accept[i]
        seqs, tables = [], []
        for n, a in zip(lens, accept):
            seq = Sequence(list(range(n + a + 1)))
            seq.block_table = rng.sample(range(5000), -(-(n + a + k + 1) // 256))
            seqs.append(seq)
            tables.append(seq.block_table)
        pos, slots, ctx = runner._draft_step_metadata(seqs, [k] * b, k)
        opos, oslots, octx = oracle.draft_metadata(lens, vrow, acc_by_row, b, b, k - 1, tables,
                                                   256)
        assert opos.tolist() == pos.tolist(), trial
        assert oslots.tolist() == slots.tolist(), trial
        assert octx.tolist() == ctx.tolist(), trial


def test_commit_metadata_agrees_with_torch_gather_formulation():
    """The rows, tokens and last rows as a torch searchsorted / where /
    index_select chain over the verify batch (an independent formulation)
    equal the restatement's, on random accept lengths."""
    import random

    rng = random.Random(9)
    for trial in range(20):
        bs, q = rng.randrange(1, 12), rng.randrange(1, 9)
        t = bs * q
        accept = [rng.randrange(0, q) for _ in range(bs)]
        starts = [rng.randrange(0, 700) for _ in range(bs)]
        tables = [rng.sample(range(50), 4) for _ in range(bs)]
        am = [rng.randrange(0, 1000) for _ in range(t)]
        cu_q, _, pos, _, rows, ids, last = oracle.commit_metadata(starts, accept, q, am, tables,
                                                                  256, t)
        cu = torch.tensor([0] + np.cumsum([a + 1 for a in accept]).tolist())
        t_idx = torch.arange(t)
        seq = torch.searchsorted(cu[1:], t_idx, right=True)
        seq_c = seq.clamp(max=bs - 1)
        trows = seq_c * q + (t_idx - cu.index_select(0, seq_c))
        trows = torch.where(seq < bs, trows, torch.full_like(trows, -1))
        tids = torch.tensor(am).index_select(0, trows.clamp(min=0))
        assert cu_q.tolist() == cu.tolist(), trial
        assert rows.tolist() == trows.tolist(), trial
        assert ids.tolist() == tids.tolist(), trial
        assert last.tolist() == (cu[1:] - 1).tolist(), trial
        committed = [s + j for s, a in zip(starts, accept) for j in range(a + 1)]
        assert pos.tolist()[:len(committed)] == committed


# ---------------------------------------------------------------- EAGLE3 draft step

def _draft_weights(seed=0, h=256, hq=4, hkv=2, d=128, inter=512, vocab=300, nbr=True):
    from oracle.draft_oracle import DraftWeights

    g = torch.Generator().manual_seed(seed)
    r = lambda *s, std=0.05: torch.randn(*s, generator=g) * std  # noqa: E731
    n1 = lambda: 1 + r(h, std=0.1)  # noqa: E731
    return DraftWeights(embed=r(vocab, h, std=1.0), fc=r(h, 3 * h), hidden_norm=n1(),
                        input_norm=n1(), qkv=r((hq + 2 * hkv) * d, 2 * h), o=r(h, hq * d),
                        post_norm=n1(), gate_up=r(2 * inter, h), down=r(h, inter), norm=n1(),
                        lm_head=r(vocab, h), d2t=torch.zeros(vocab, dtype=torch.int64),
                        num_heads=hq, num_kv_heads=hkv, head_dim=d, eps=1e-6, rope_theta=1e6,
                        norm_before_residual=nbr)


def _llama_config(w):
    from transformers import LlamaConfig

    h = w.embed.shape[1]
    return LlamaConfig(hidden_size=h, intermediate_size=w.down.shape[1],
                       num_attention_heads=w.num_heads, num_key_value_heads=w.num_kv_heads,
                       head_dim=w.head_dim, rope_theta=w.rope_theta, rms_norm_eps=w.eps,
                       max_position_embeddings=8192)


def test_draft_oracle_norm_rope_mlp_match_transformers_llama():
    """The restatement's RMSNorm, neox RoPE and gated MLP against the
    transformers Llama modules (float32): an independent implementation of
    the same published layer (the EAGLE3 draft layer is Llama-style)."""
    from transformers.models.llama.modeling_llama import (LlamaMLP, LlamaRMSNorm,
                                                          LlamaRotaryEmbedding,
                                                          apply_rotary_pos_emb)

    from oracle import draft_oracle as D

    w = _draft_weights()
    cfg = _llama_config(w)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(7, 256, generator=g) * 3
    ln = LlamaRMSNorm(256, eps=1e-6)
    ln.weight.data.copy_(w.hidden_norm)
    torch.testing.assert_close(D.rms_norm(x, w.hidden_norm, 1e-6), ln(x), rtol=1e-6, atol=1e-6)
    rot = LlamaRotaryEmbedding(cfg)
    q = torch.randn(4, 128, generator=g)
    for pos in (0, 1, 37, 4095):
        cos, sin = rot(q[None], torch.tensor([[pos]]))
        ref, _ = apply_rotary_pos_emb(q[None, :, None, :], q[None, :, None, :], cos, sin)
        torch.testing.assert_close(D.rope(q, pos, w.rope_theta), ref[0, :, 0], rtol=1e-5,
                                   atol=2e-5)
    m = LlamaMLP(cfg)
    m.gate_proj.weight.data.copy_(w.gate_up[:512])
    m.up_proj.weight.data.copy_(w.gate_up[512:])
    m.down_proj.weight.data.copy_(w.down)
    with torch.no_grad():
        torch.testing.assert_close(D.mlp(w, x[0]), m(x[:1])[0], rtol=1e-5, atol=1e-6)


def test_draft_oracle_attention_matches_sdpa_and_closed_forms():
    """attend() equals torch's scaled_dot_product_attention over the same
    keys with GQA; a single visible key returns its V row; equal scores
    return the mean of the V rows."""
    import torch.nn.functional as F

    from oracle import draft_oracle as D

    g = torch.Generator().manual_seed(2)
    q = torch.randn(8, 128, generator=g)
    k = torch.randn(50, 2, 128, generator=g)
    v = torch.randn(50, 2, 128, generator=g)
    kk = k.repeat_interleave(4, 1).permute(1, 0, 2)[None]       # [1, Hq, n, D]
    vv = v.repeat_interleave(4, 1).permute(1, 0, 2)[None]
    ref = F.scaled_dot_product_attention(q[None, :, None, :], kk, vv)[0, :, 0]
    torch.testing.assert_close(D.attend(q, k, v), ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(D.attend(q, k[:1], v[:1]), v[0].repeat_interleave(4, 0))
    flat = torch.zeros(8, 128)
    torch.testing.assert_close(D.attend(flat, k, v), v.mean(0).repeat_interleave(4, 0))


@pytest.mark.parametrize("nbr", [True, False])
def test_draft_oracle_layer_and_recurrence_closed_forms(nbr):
    """With zero attention and MLP output projections the draft layer passes
    its residual through: the pre-norm state is hidden_norm(h) when the norm
    comes before the residual (eagle3.py:133-135), h itself otherwise, and
    the sampled state is its final norm.  Then every proposal after the
    first is the same token (the fed-back state is a fixed point of the
    normalisation), and a commit's state depends on fc of the last aux row
    only."""
    from oracle import draft_oracle as D

    w = _draft_weights(nbr=nbr)
    w.o.zero_()
    w.down.zero_()
    g = torch.Generator().manual_seed(3)
    h = torch.randn(256, generator=g)
    hist = torch.randn(5, 2, 128, generator=g)
    normed, pre, k, v = D.forward_token(w, 17, 5, h, hist, hist)
    want_pre = D.rms_norm(h, w.hidden_norm, w.eps) if nbr else h
    torch.testing.assert_close(pre, want_pre)
    torch.testing.assert_close(normed, D.rms_norm(want_pre, w.norm, w.eps))
    # the new V row is the value projection of [norm(embed) | norm(h)]
    attn_in = torch.cat((D.rms_norm(w.embed[17], w.input_norm, w.eps),
                         D.rms_norm(h, w.hidden_norm, w.eps)))
    torch.testing.assert_close(v, (w.qkv[(4 + 2) * 128:] @ attn_in).view(2, 128))
    if nbr:
        w.hidden_norm.fill_(1.0)
        toks, rows, ks, vs = D.propose(w, D.rms_norm(h, w.norm, w.eps), h, 5, 4, hist, hist)
        assert len(set(toks[1:])) == 1 and ks.shape == (3, 2, 128)
        fixed = D.rms_norm(D.rms_norm(h, w.hidden_norm, w.eps), w.norm, w.eps)
        assert toks[1] == int(torch.argmax(w.lm_head @ fixed))
    aux = torch.randn(3, 768, generator=g)
    n1, p1, ks, _ = D.commit(w, [3, 9, 11], aux, 5, hist, hist)
    n2, p2, _, _ = D.commit(w, [40, 9, 11], torch.cat((torch.randn(2, 768, generator=g),
                                                       aux[2:])), 5, hist, hist)
    torch.testing.assert_close(p1, p2)
    assert ks.shape == (3, 2, 128)


def test_draft_oracle_sampling_maps_through_d2t():
    """sample_greedy returns argmax + d2t[argmax] (eagle3.py:294-296)."""
    from oracle import draft_oracle as D

    w = _draft_weights()
    w.lm_head.zero_()
    x = torch.ones(256)
    w.lm_head[123] = 1.0                      # argmax row 123
    w.d2t[123] = 1000
    assert D.sample_greedy(w, x) == 1123
    w.lm_head[200] = 1.0                      # a tie: the first index wins
    assert D.sample_greedy(w, x) == 1123
