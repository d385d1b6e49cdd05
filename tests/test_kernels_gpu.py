"""GPU parity of the four hot-path kernels against the CPU oracle.

Integer / byte work (argmax, accept, KV store, rollback, aux gather) must be
bit-exact; attention must be within 2e-2 max-abs of the double-precision
textbook result and FP8 decode within 2e-3 (the
reference's own bound, tests/test_fp8_kv_cache.py:81 of the reference).
Every call goes through the C ABI (nanovllm_amd.kernels -> libnanovllm_amd.so).
"""
import numpy as np
import pytest
import torch

from helpers import acceptance_logits, bits, paged_case
from oracle import oracle

pytestmark = pytest.mark.gpu

ATTN_TOL = 2e-2
FP8_TOL = 2e-3


@pytest.fixture(scope="module")
def K(cuda):
    from nanovllm_amd import kernels

    return kernels


# ---------------------------------------------------------------- K4

@pytest.mark.parametrize("batch,k,vocab,seed", [(8, 4, 151936, 0), (64, 5, 151936, 2),
                                                 (3, 8, 1000, 5), (5, 1, 37, 6)])
def test_argmax_accept_matches_oracle(K, cuda, batch, k, vocab, seed):
    logits, cu_q, ids, _ = acceptance_logits(batch, k, vocab, 0.7, seed)
    am, acc, bonus = K.argmax_accept(logits.to(cuda), cu_q.to(cuda), ids.to(cuda))
    torch.cuda.synchronize()
    ref_am = oracle.argmax_bf16(bits(logits))
    ref_acc, ref_bonus = oracle.accept(cu_q.numpy(), ref_am, ids.numpy())
    np.testing.assert_array_equal(am.cpu().numpy(), ref_am)
    np.testing.assert_array_equal(acc.cpu().numpy(), ref_acc)
    np.testing.assert_array_equal(bonus.cpu().numpy(), ref_bonus)
    # and the torch reference semantics on the same bytes
    np.testing.assert_array_equal(ref_am, logits.argmax(-1).numpy())


def test_argmax_accept_on_the_committed_config1_fixture(K, cuda):
    """K4 on BASELINE config 1's committed reduced-vocabulary fixture
    (tests/golden/config1_reduced.npz), against its frozen outputs."""
    import os
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "config1_reduced.npz"))
    logits = torch.from_numpy(f["logits_bits"].view(np.int16)).view(torch.bfloat16).to(cuda)
    am, acc, bonus = K.argmax_accept(logits, torch.from_numpy(f["cu_q"]).to(cuda),
                                     torch.from_numpy(f["input_ids"]).to(cuda))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(am.cpu().numpy(), f["argmax"])
    np.testing.assert_array_equal(acc.cpu().numpy(), f["accept_len"])
    np.testing.assert_array_equal(bonus.cpu().numpy(), f["bonus"])


@pytest.mark.parametrize("layout", ["odd_width", "aligned", "padded_rows"])
def test_argmax_edge_values(K, cuda, layout):
    """NaN / signed zero / inf / denormal / tie cases on both partial kernels:
    an odd row width takes the element-wise kernel, 16-byte aligned rows the
    register-resident vector kernel (with and without a tail of elements
    past the last whole vector)."""
    v = 70008 if layout == "aligned" else 70001
    g = torch.Generator().manual_seed(11)
    x = torch.randn(10, v, generator=g).to(torch.bfloat16)
    xb = x.view(torch.int16)
    x[0, 100] = 50.0
    x[0, 60000] = 50.0                       # tie across chunks: first index wins
    xb[1, 5000] = 0x7FC1                     # NaN beats everything
    xb[1, 70000] = -64                       # 0xFFC0 negative NaN, later (tail element)
    x[2, :] = -1.0
    x[2, 777] = -0.0
    x[2, 778] = 0.0                          # -0 == +0 -> first
    x[3, :] = float("-inf")                  # all -inf -> 0
    x[4, :] = 3.0                            # all equal -> 0
    x[5, 70000] = 1e30                       # max at the tail element
    x[6, 0] = float("inf")
    xb[7, 69999] = 0x7F80                    # +inf late
    x[7, 3] = 3e38
    x[8, :] = -1.0
    xb[8, 50] = 0x0000
    xb[8, 123] = 0x0001                      # smallest positive denormal beats +0
    xb[9, :] = -32767                        # 0x8001: negative denormals
    xb[9, 4000] = -32768                     # 0x8000: -0
    xb[9, 6000] = 0x0000                     # +0 ties -0: first
    cu = torch.tensor([0, 3, 8, 10], dtype=torch.int32)
    ids = torch.zeros(10, dtype=torch.int64)
    if layout == "padded_rows":
        wide = torch.full((10, 70016), -1.0, dtype=torch.bfloat16)
        wide[:, :v] = x
        dx = wide.to(cuda)[:, :v]            # row stride 70016: 16-byte aligned rows
    else:
        dx = x.to(cuda)
    am, acc, bonus = K.argmax_accept(dx, cu.to(cuda), ids.to(cuda))
    ref = oracle.argmax_bf16(bits(x))
    np.testing.assert_array_equal(ref, x.argmax(-1).numpy())
    np.testing.assert_array_equal(am.cpu().numpy(), ref)
    ra, rb = oracle.accept(cu.numpy(), ref, ids.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), ra)
    np.testing.assert_array_equal(bonus.cpu().numpy(), rb)


def test_argmax_vector_kernel_random_rows(K, cuda):
    """Aligned rows of several widths (one chunk, many chunks, a short tail):
    the vector kernel against the oracle and torch on the same bytes."""
    g = torch.Generator().manual_seed(12)
    for v in (8, 2048, 4104, 32768, 151936, 151943):
        rows = 37
        x = torch.randn(rows, v, generator=g).to(torch.bfloat16)
        # repeated maxima inside one vector and across threads
        x[0, : min(v, 16)] = 9.0
        x[1, v // 2:] = 9.0
        wide = torch.zeros(rows, (v + 7) // 8 * 8, dtype=torch.bfloat16)
        wide[:, :v] = x
        out = K.argmax_rows(wide.to(cuda)[:, :v])
        ref = oracle.argmax_bf16(bits(x)).astype(np.int64)
        np.testing.assert_array_equal(ref, x.argmax(-1).numpy())
        np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"vocab {v}")


def test_argmax_accept_ragged_and_empty(K, cuda):
    g = torch.Generator().manual_seed(3)
    qs = [1, 9, 0, 4, 2, 0, 6]
    t = sum(qs)
    vocab = 5000
    logits = torch.randn(t, vocab, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0] + np.cumsum(qs).tolist(), dtype=torch.int32)
    ref_am = oracle.argmax_bf16(bits(logits))
    ids = torch.randint(0, vocab, (t,), generator=g)
    # make some proposals match so accept lengths vary
    for i, q in enumerate(qs):
        s = int(cu[i])
        for j in range(q - 1):
            if (i + j) % 3 != 2:
                ids[s + 1 + j] = int(ref_am[s + j])
    am, acc, bonus = K.argmax_accept(logits.to(cuda), cu.to(cuda), ids.to(cuda))
    ra, rb = oracle.accept(cu.numpy(), ref_am, ids.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), ra)
    np.testing.assert_array_equal(bonus.cpu().numpy(), rb)
    assert rb[2] == -1 and ra[2] == 0


def test_argmax_accept_graph_replay(K, cuda):
    """Self-resetting counters: replaying a captured call stays correct."""
    logits, cu_q, ids, _ = acceptance_logits(16, 5, 151936, 0.7, 9)
    dl, dcu, dids = logits.to(cuda), cu_q.to(cuda), ids.to(cuda)
    out = torch.empty(logits.shape[0] + 32, dtype=torch.int32, device=cuda)
    K.argmax_accept(dl, dcu, dids, out=out)           # grows the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        K.argmax_accept(dl, dcu, dids, out=out)
    for rep in range(4):
        nl, ncu, nids, _ = acceptance_logits(16, 5, 151936, 0.5, 100 + rep)
        dl.copy_(nl)
        dids.copy_(nids)
        out.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        ref = oracle.argmax_bf16(bits(nl))
        ra, rb = oracle.accept(ncu.numpy(), ref, nids.numpy())
        got = out.cpu().numpy()
        t = nl.shape[0]
        np.testing.assert_array_equal(got[:t], ref)
        np.testing.assert_array_equal(got[t:t + 16], ra)
        np.testing.assert_array_equal(got[t + 16:], rb)
        # eager work between replays
        K.argmax_accept(dl, dcu, dids)
        torch.cuda.synchronize()


@pytest.mark.parametrize("shape", ["many_chunks", "multi_pass", "wave_per_sequence"])
def test_argmax_finalize_passes(K, cuda, shape):
    """Both merge kernels.  Up to 8192 chunk keys go through the one-workgroup
    merge: rows split into more than 16 chunks, and long sequences with the
    accepted prefix running far into them.  Beyond that (here 8400 keys) the
    wave-per-sequence merge loads the keys of as many rows as a wave's lanes
    hold per pass, with the accepted prefix running across pass boundaries."""
    g = torch.Generator().manual_seed(21)
    if shape == "many_chunks":
        qs, vocab = [3, 1], 300000            # 19 chunks of 16384 elements per row
    elif shape == "multi_pass":
        qs, vocab = [30, 27, 9, 30], 32768    # two chunks per row
    else:                                     # 840 rows x 10 chunks: past the one-workgroup limit
        qs, vocab = [30, 27, 9, 30] + [6] * 124, 151936
    t = sum(qs)
    logits = torch.randn(t, vocab, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0] + np.cumsum(qs).tolist(), dtype=torch.int32)
    ref_am = oracle.argmax_bf16(bits(logits))
    np.testing.assert_array_equal(ref_am, logits.argmax(-1).numpy())
    ids = torch.randint(0, vocab, (t,), generator=g)
    # accept every proposal up to a per-sequence row, then reject
    stops = ([2, 0, 8, 29] + [i % 6 for i in range(len(qs))])[: len(qs)]
    for i, q in enumerate(qs):
        s = int(cu[i])
        for j in range(min(stops[i], q - 1)):
            ids[s + 1 + j] = int(ref_am[s + j])
        if stops[i] < q - 1:
            ids[s + 1 + stops[i]] = (int(ref_am[s + stops[i]]) + 1) % vocab
    am, acc, bonus = K.argmax_accept(logits.to(cuda), cu.to(cuda), ids.to(cuda))
    ra, rb = oracle.accept(cu.numpy(), ref_am, ids.numpy())
    np.testing.assert_array_equal(am.cpu().numpy(), ref_am)
    np.testing.assert_array_equal(acc.cpu().numpy(), ra)
    np.testing.assert_array_equal(bonus.cpu().numpy(), rb)
    assert ra.tolist() == [min(s_, q - 1) for s_, q in zip(stops, qs)]
    out = K.argmax_rows(logits.to(cuda))
    np.testing.assert_array_equal(out.cpu().numpy(), ref_am.astype(np.int64))


def test_argmax_rows_with_index_map(K, cuda):
    g = torch.Generator().manual_seed(4)
    rows, vocab = 64, 32000
    logits = torch.randn(rows, vocab, generator=g).to(torch.bfloat16)
    d2t = torch.randint(-5, 100, (vocab,), generator=g)
    out = K.argmax_rows(logits.to(cuda), d2t.to(cuda))
    ref = oracle.argmax_bf16(bits(logits)).astype(np.int64)
    np.testing.assert_array_equal(out.cpu().numpy(), ref + d2t.numpy()[ref])
    out2 = K.argmax_rows(logits.to(cuda))
    np.testing.assert_array_equal(out2.cpu().numpy(), ref)


# ---------------------------------------------------------------- K2

@pytest.mark.parametrize("layout", ["token_major", "head_major", "rows_entry"])
@pytest.mark.parametrize("fp8", [False, True])
def test_store_kvcache_matches_oracle(K, cuda, fp8, layout):
    g = torch.Generator().manual_seed(21)
    t, hq, hkv, d, nb, bs = 160, 16, 8, 128, 12, 256
    # key/value as views into a fused QKV output (row stride > row)
    qkv = (torch.randn(t, (hq + 2 * hkv) * d, generator=g) * 0.5).to(torch.bfloat16)
    key = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    value = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    slots = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    slots[::7] = -1
    cdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    init = (torch.randn(nb, bs, hkv, d, generator=g)).to(cdt)
    if layout == "head_major":
        # pages stored [nb, Hkv, bs, D], passed as a [nb, bs, Hkv, D] view
        kc = init.permute(0, 2, 1, 3).contiguous().to(cuda).permute(0, 2, 1, 3)
        vc = init.permute(0, 2, 1, 3).contiguous().to(cuda).permute(0, 2, 1, 3)
    else:
        kc, vc = init.clone().to(cuda), init.clone().to(cuda)
    ks = torch.tensor([1.0], device=cuda) if fp8 else None
    dq = qkv.to(cuda)
    store = K.store_kvcache_rows if layout == "rows_entry" else K.store_kvcache
    store(dq[:, hq * d:(hq + hkv) * d].view(t, hkv, d),
          dq[:, (hq + hkv) * d:].view(t, hkv, d), kc, vc, slots.to(cuda), ks, ks)
    kc, vc = kc.contiguous(), vc.contiguous()
    rk, rv = bits(init).copy(), bits(init).copy()
    oracle.store_kv(bits(key.contiguous()), bits(value.contiguous()), rk, rv, slots.numpy())
    np.testing.assert_array_equal(bits(kc.cpu()), rk)
    np.testing.assert_array_equal(bits(vc.cpu()), rv)


def test_store_kvcache_fp8_scale_and_saturation(K, cuda):
    vals = torch.tensor([0.0, -0.0, 1e-4, 0.0009765625, 0.0017, 0.3, -2.5, 447.0, 463.9, 464.0,
                         465.0, 1e6, -1e6, float("inf"), float("-inf"), 240.0],
                        dtype=torch.float32)
    d = 128
    row = torch.zeros(1, 1, d)
    row[0, 0, :vals.numel()] = vals
    key = row.to(torch.bfloat16)
    value = (row * 0.5).to(torch.bfloat16)
    kc = torch.zeros(1, 256, 1, d, dtype=torch.float8_e4m3fn, device=cuda)
    vc = torch.zeros_like(kc)
    slot = torch.tensor([5], dtype=torch.int32, device=cuda)
    ks = torch.tensor([0.5], device=cuda)
    vs = torch.tensor([2.0], device=cuda)
    K.store_kvcache(key.to(cuda), value.to(cuda), kc, vc, slot, ks, vs)
    rk = np.zeros((1, 256, 1, d), np.uint8)
    rv = np.zeros((1, 256, 1, d), np.uint8)
    oracle.store_kv(bits(key), bits(value), rk, rv, np.array([5], np.int32), 0.5, 2.0)
    np.testing.assert_array_equal(bits(kc.cpu()), rk)
    np.testing.assert_array_equal(bits(vc.cpu()), rv)


@pytest.mark.parametrize("poison", [False, True])
def test_rollback_matches_oracle(K, cuda, poison):
    g = torch.Generator().manual_seed(8)
    qs = [5, 5, 1, 6, 3]
    cu = torch.tensor([0] + np.cumsum(qs).tolist(), dtype=torch.int32)
    t = int(cu[-1])
    acc = torch.tensor([0, 4, 0, 2, 7], dtype=torch.int32)   # 7 is clamped to q-1
    slots = torch.randperm(4 * 256, generator=g)[:t].to(torch.int32)
    lens = torch.tensor([900, 33, 12, 600, 70], dtype=torch.int32)
    layers = 3
    cache = torch.randn(2, layers, 4, 256, 2, 128, generator=g).to(torch.bfloat16)
    dcache = cache.to(cuda)
    dslots, dlens = slots.to(cuda), lens.to(cuda)
    K.rollback(cu.to(cuda), acc.to(cuda), dslots, dlens, dcache[0], dcache[1], poison=poison)
    rk, rv = bits(cache[0]).copy(), bits(cache[1]).copy()
    rs, rl = slots.numpy(), lens.numpy()
    for layer in range(layers):
        s2, l2 = oracle.rollback(cu.numpy(), acc.numpy(), rs, rl, rk[layer], rv[layer], poison)
    np.testing.assert_array_equal(dslots.cpu().numpy(), s2)
    np.testing.assert_array_equal(dlens.cpu().numpy(), l2)
    np.testing.assert_array_equal(bits(dcache[0].cpu()), rk)
    np.testing.assert_array_equal(bits(dcache[1].cpu()), rv)


# ---------------------------------------------------------------- K3

def test_aux_gather_matches_oracle(K, cuda):
    g = torch.Generator().manual_seed(13)
    t, h = 384, 4096
    hid = [(torch.randn(t, h, generator=g) * (10 ** i)).to(torch.bfloat16) for i in range(3)]
    res = [(torch.randn(t, h, generator=g) * 3).to(torch.bfloat16) for _ in range(3)]
    hid[1][5, :4] = torch.tensor([float("inf"), float("nan"), 1e38, -1e38])
    res[1][5, :4] = torch.tensor([float("-inf"), 1.0, 1e38, -1e38])
    src = torch.randint(0, t, (100,), generator=g).to(torch.int32)
    src[3] = -1
    out = K.aux_gather([x.to(cuda) for x in hid], [x.to(cuda) for x in res], src.to(cuda))
    ref = oracle.aux_gather([bits(x) for x in hid], [bits(x) for x in res],
                            np.maximum(src.numpy(), 0))
    ref[3] = 0
    np.testing.assert_array_equal(bits(out.cpu()), ref)


# ---------------------------------------------------------------- K1

def _run_verify(K, cuda, case, fp8=False, head_major=False):
    kc = case["k_cache"].clone()
    vc = case["v_cache"].clone()
    if fp8:
        kc = kc.float().to(torch.float8_e4m3fn)
        vc = vc.float().to(torch.float8_e4m3fn)
    if head_major == "kv_adjacent":
        # the engine's pages: [blocks, Hkv, 2, block_size, D] (a head's K rows
        # then its V rows), K and V seen as [blocks, block_size, Hkv, D]
        both = torch.stack([kc.permute(0, 2, 1, 3), vc.permute(0, 2, 1, 3)], 2).contiguous()
        both = both.to(cuda).permute(2, 0, 3, 1, 4)
        dkc, dvc = both[0], both[1]
    elif head_major:
        # pages stored [blocks, Hkv, block_size, D], seen as [blocks, block_size, Hkv, D]
        dkc = kc.permute(0, 2, 1, 3).contiguous().to(cuda).permute(0, 2, 1, 3)
        dvc = vc.permute(0, 2, 1, 3).contiguous().to(cuda).permute(0, 2, 1, 3)
    else:
        dkc, dvc = kc.to(cuda), vc.to(cuda)
    one = torch.ones(1, device=cuda) if fp8 else None
    K.store_kvcache(case["k_new"].to(cuda), case["v_new"].to(cuda), dkc, dvc,
                    case["slot_mapping"].to(cuda), one, one)
    hq = case["q"].shape[1]
    d = case["q"].shape[2]
    out = K.paged_attention_varlen(
        case["q"].to(cuda), dkc, dvc, case["cu_q"].to(cuda), case["cu_k"].to(cuda),
        max(case["q_lens"]), int(case["lens"].max()), d ** -0.5, case["block_tables"].to(cuda),
        k_scale=one, v_scale=one)
    torch.cuda.synchronize()
    # oracle: store then attention on the CPU copy
    rk, rv = bits(kc).copy(), bits(vc).copy()
    oracle.store_kv(bits(case["k_new"]), bits(case["v_new"]), rk, rv, case["slot_mapping"].numpy())
    np.testing.assert_array_equal(bits(dkc.contiguous().cpu()), rk)
    ref = oracle.paged_attention(bits(case["q"]), rk, rv, case["cu_q"].numpy(),
                                 case["lens"].numpy(), case["block_tables"].numpy(), d ** -0.5)
    got = out.float().cpu().numpy()
    return got, ref


@pytest.mark.parametrize("name,kw", [
    ("config2", dict(seed=1, batch=32, q_len=5, ctx_lo=512, ctx_hi=4096, hq=16, hkv=8)),
    ("gqa4_k5", dict(seed=2, batch=6, q_len=6, ctx_lo=20, ctx_hi=1500, hq=32, hkv=8)),
    ("gqa8_k7", dict(seed=3, batch=4, q_len=8, ctx_lo=8, ctx_hi=900, hq=64, hkv=8)),
    # 64-row tiles over 3500-8000 keys: several splits per tile plus the combine
    ("gqa8_k7_long", dict(seed=16, batch=6, q_len=8, ctx_lo=3500, ctx_hi=8000, hq=64, hkv=8)),
    ("ragged", dict(seed=4, batch=7, q_len=[1, 3, 6, 2, 5, 4, 1], ctx_lo=1, ctx_hi=700, hq=16,
                    hkv=4)),
    ("short", dict(seed=5, batch=5, q_len=3, ctx_lo=3, ctx_hi=40, hq=8, hkv=8)),
])
def test_verify_attention_bf16(K, cuda, name, kw):
    got, ref = _run_verify(K, cuda, paged_case(**kw))
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL, (name, err)


@pytest.mark.parametrize("block_size", [32, 64, 128])
@pytest.mark.parametrize("name,kw,fp8", [
    # eight waves per split; with small pages a split holds at most 62 pages,
    # so long sequences take several splits and the combine
    ("q6_gqa4", dict(seed=30, batch=8, q_len=6, ctx_lo=30, ctx_hi=3000, hq=32, hkv=8), False),
    # FP8 stream ranges across page boundaries
    ("q5_gqa2_fp8", dict(seed=31, batch=10, q_len=5, ctx_lo=40, ctx_hi=2600, hq=16, hkv=8), True),
    # 64-row tiles, one wave per split
    ("q8_gqa8", dict(seed=32, batch=4, q_len=8, ctx_lo=100, ctx_hi=2500, hq=64, hkv=8), False),
    ("decode", dict(seed=33, batch=10, q_len=1, ctx_lo=1, ctx_hi=2000, hq=32, hkv=8), False),
])
def test_verify_attention_small_pages(K, cuda, block_size, name, kw, fp8):
    """Pages of 32, 64 and 128 tokens (the ABI takes any multiple of 32): the
    same store + attention against the oracle, so the per-split page limit,
    the chunk-to-page addressing and the combine hold off the 256-token
    default too."""
    case = paged_case(block_size=block_size, **kw)
    got, ref = _run_verify(K, cuda, case, fp8=fp8)
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL, (name, block_size, err)


@pytest.mark.parametrize("name,kw", [
    # paired mode (17-32-row single tiles, more than one and at most two
    # (sequence, kv head) pairs per CU of a 256-CU device): grid rows past
    # CUs / Hkv take the sequences from the last one backwards
    ("hkv4_b100", dict(seed=40, batch=100, q_len=6, ctx_lo=20, ctx_hi=400, hq=16, hkv=4)),
    # 264 pairs: a single reversed row, which maps to itself
    ("b33_q5", dict(seed=41, batch=33, q_len=5, ctx_lo=30, ctx_hi=500, hq=32, hkv=8)),
    ("ragged_b40", dict(seed=42, batch=40, q_len=[1, 7, 3, 6, 2, 5, 4, 7] * 5, ctx_lo=1,
                        ctx_hi=600, hq=32, hkv=8)),
    # whole-sequence splits up to the mode's 3072-key bound
    ("long_b36", dict(seed=43, batch=36, q_len=6, ctx_lo=2900, ctx_hi=3072, hq=32, hkv=8)),
    # 32-token pages: a whole-sequence split would span more pages than a
    # wave holds block ids, so the launch falls back to eight-wave splits
    ("pages32_b40", dict(seed=44, batch=40, q_len=6, ctx_lo=2000, ctx_hi=3000, hq=32, hkv=8,
                         block_size=32)),
])
def test_verify_attention_paired_geometries(K, cuda, name, kw):
    """The paired decomposition's row mapping and its fallback, against the
    oracle, on batches in drawn order (the mapping is a permutation of the
    sequences whatever their order)."""
    got, ref = _run_verify(K, cuda, paged_case(**kw))
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL, (name, err)


def test_verify_attention_paired_with_empty_padding_sequences(K, cuda):
    """A verify graph's bucket pads the batch with empty sequences (no query
    rows, no keys) after the real ones; in paired mode those take grid rows
    among the reversed ones.  40 real sequences of 24-row tiles padded to
    64 (512 (sequence, kv head) pairs): the real rows against the oracle."""
    case = paged_case(seed=45, batch=40, q_len=6, ctx_lo=50, ctx_hi=1500, hq=32, hkv=8)
    pad = 24
    cu_q = torch.cat([case["cu_q"], case["cu_q"][-1:].repeat(pad)])
    cu_k = torch.cat([case["cu_k"], case["cu_k"][-1:].repeat(pad)])
    bt = torch.cat([case["block_tables"],
                    torch.full((pad, case["block_tables"].shape[1]), -1, dtype=torch.int32)])
    kc, vc = case["k_cache"].to(cuda), case["v_cache"].to(cuda)
    K.store_kvcache(case["k_new"].to(cuda), case["v_new"].to(cuda), kc, vc,
                    case["slot_mapping"].to(cuda), None, None)
    out = K.paged_attention_varlen(case["q"].to(cuda), kc, vc, cu_q.to(cuda), cu_k.to(cuda), 6,
                                   int(case["lens"].max()), 128 ** -0.5, bt.to(cuda))
    torch.cuda.synchronize()
    rk, rv = bits(case["k_cache"]).copy(), bits(case["v_cache"]).copy()
    oracle.store_kv(bits(case["k_new"]), bits(case["v_new"]), rk, rv, case["slot_mapping"].numpy())
    ref = oracle.paged_attention(bits(case["q"]), rk, rv, case["cu_q"].numpy(),
                                 case["lens"].numpy(), case["block_tables"].numpy(), 128 ** -0.5)
    err = np.abs(out.float().cpu().numpy() - ref).max()
    assert err <= ATTN_TOL, err


def test_verify_attention_fp8(K, cuda):
    case = paged_case(seed=7, batch=8, q_len=5, ctx_lo=300, ctx_hi=3000, hq=16, hkv=8)
    got, ref = _run_verify(K, cuda, case, fp8=True)
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL, err


@pytest.mark.parametrize("name,kw", [
    # more sequences than the stream decomposition takes (8 x 64): the fixed
    # FP8 path with its K rows staged, 4-row tiles (one column tile) and
    # 20-row tiles (two); 32-token pages keep the cache small
    ("fp8_fixed_4rows", dict(seed=40, batch=520, q_len=2, ctx_lo=2, ctx_hi=100, hq=4, hkv=2,
                             block_size=32)),
    ("fp8_fixed_20rows", dict(seed=41, batch=520, q_len=5, ctx_lo=5, ctx_hi=100, hq=8, hkv=2,
                              block_size=32)),
])
def test_verify_attention_fp8_fixed_decomposition(K, cuda, name, kw):
    got, ref = _run_verify(K, cuda, paged_case(**kw), fp8=True)
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL, (name, err)


@pytest.mark.parametrize("pages", ["head_major", "kv_adjacent"])
@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("name,kw", [
    ("config3", dict(seed=8, batch=16, q_len=6, ctx_lo=256, ctx_hi=2304, hq=32, hkv=8)),
    ("decode", dict(seed=9, batch=12, q_len=1, ctx_lo=1, ctx_hi=1200, hq=32, hkv=8)),
    ("gqa8_k7", dict(seed=10, batch=3, q_len=8, ctx_lo=8, ctx_hi=900, hq=64, hkv=8)),
])
def test_verify_attention_head_major_pages(K, cuda, name, kw, fp8, pages):
    """Head-major pages ([blocks, Hkv, block_size, D] storage, and the
    engine's [blocks, Hkv, 2, block_size, D] with a head's K and V rows
    adjacent): the same store + attention through strided views."""
    got, ref = _run_verify(K, cuda, paged_case(**kw), fp8=fp8, head_major=pages)
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL, (name, fp8, pages, err)


def test_fp8_decode_reference_geometry(K, cuda):
    """The reference's FP8 test geometry (tests/test_fp8_kv_cache.py:20-41 of
    the reference): 300 tokens, 2 blocks of 256 in table order [1, 0], 4 q /
    2 kv heads, D=128.  Store -> page round trip is exact; decode matches the
    fp32 einsum softmax within 2e-3; a captured graph re-reads a device-side
    context length (113, then 300)."""
    torch.manual_seed(0)
    length, bs, hkv, hq, d = 300, 256, 2, 4, 128
    key = (torch.randn(length, hkv, d) * 0.1).to(torch.bfloat16)
    value = (torch.randn(length, hkv, d) * 0.1).to(torch.bfloat16)
    kc = torch.empty(2, bs, hkv, d, dtype=torch.float8_e4m3fn, device=cuda)
    vc = torch.empty_like(kc)
    table = torch.tensor([[1, 0]], dtype=torch.int32, device=cuda)
    pos = torch.arange(length, device=cuda)
    slots = (table[0, pos // bs] * bs + pos % bs).to(torch.int32)
    scale = torch.ones(1, device=cuda)
    K.store_kvcache(key.to(cuda), value.to(cuda), kc, vc, slots, scale, scale)
    qk = kc[table[0].long()].reshape(-1, hkv, d)[:length].cpu()
    qv = vc[table[0].long()].reshape(-1, hkv, d)[:length].cpu()
    np.testing.assert_array_equal(bits(qk), oracle.f32_to_e4m3(key.float().numpy()))
    np.testing.assert_array_equal(bits(qv), oracle.f32_to_e4m3(value.float().numpy()))
    query = (torch.randn(1, hq, d) * 0.1).to(torch.bfloat16)

    def ref_for(n):
        ek = qk[:n].float().repeat_interleave(hq // hkv, dim=1)
        ev = qv[:n].float().repeat_interleave(hq // hkv, dim=1)
        w = torch.softmax(torch.einsum("hd,lhd->hl", query[0].float(), ek) * d ** -0.5, -1)
        return torch.einsum("hl,lhd->hd", w, ev)

    actual = K.fp8_paged_decode_attention(query.to(cuda), kc, vc,
                                          torch.tensor([length], dtype=torch.int32, device=cuda),
                                          table, d ** -0.5, scale, scale)
    assert (actual[0].float().cpu() - ref_for(length)).abs().max().item() <= FP8_TOL
    # restated reference kernel agrees too
    rest = oracle.fp8_paged_decode(bits(query), bits(kc.cpu()), bits(vc.cpu()),
                                   np.array([length], np.int32), table.cpu().numpy(), d ** -0.5)
    assert np.abs(rest[0] - ref_for(length).numpy()).max() <= FP8_TOL

    ctx = torch.ones(1, dtype=torch.int32, device=cuda)
    dq = query.to(cuda)
    K.fp8_paged_decode_attention(dq, kc, vc, ctx, table, d ** -0.5, scale, scale)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout = K.fp8_paged_decode_attention(dq, kc, vc, ctx, table, d ** -0.5, scale, scale)
    for n in (113, length, 1, 256):
        ctx.fill_(n)
        graph.replay()
        torch.cuda.synchronize()
        assert (gout[0].float().cpu() - ref_for(n)).abs().max().item() <= FP8_TOL, n


def test_decode_matches_varlen_single_row(K, cuda):
    case = paged_case(seed=12, batch=9, q_len=1, ctx_lo=1, ctx_hi=2100, hq=32, hkv=8)
    got, ref = _run_verify(K, cuda, case)
    assert np.abs(got - ref).max() <= ATTN_TOL
    # decode entry on the same cache state: identical math path
    dkc = case["k_cache"].clone().to(cuda)
    dvc = case["v_cache"].clone().to(cuda)
    K.store_kvcache(case["k_new"].to(cuda), case["v_new"].to(cuda), dkc, dvc,
                    case["slot_mapping"].to(cuda))
    out = K.paged_attention_decode(case["q"].to(cuda), dkc, dvc, case["lens"].to(cuda),
                                   case["block_tables"].to(cuda), 128 ** -0.5)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATTN_TOL


def test_attention_skips_invalid_block_ids(K, cuda):
    """Block-table entries outside [0, num_blocks) are treated as empty."""
    case = paged_case(seed=14, batch=3, q_len=2, ctx_lo=300, ctx_hi=600, hq=8, hkv=2)
    bt = case["block_tables"].clone()
    nb = case["k_cache"].shape[0]
    # first block of sequence 0 becomes invalid -> its keys are masked
    bt[0, 0] = nb + 100
    kc, vc = case["k_cache"].to(cuda), case["v_cache"].to(cuda)
    out = K.paged_attention_varlen(case["q"].to(cuda), kc, vc, case["cu_q"].to(cuda),
                                   case["cu_k"].to(cuda), 2, int(case["lens"].max()), 128 ** -0.5,
                                   bt.to(cuda))
    torch.cuda.synchronize()
    # reference: mask = drop keys [0, 256) of sequence 0 by pointing them at
    # an all-zero score... compute directly in numpy
    q = case["q"].float().numpy()
    kcf = case["k_cache"].float().numpy()
    vcf = case["v_cache"].float().numpy()
    L = int(case["lens"][0])
    keys = np.stack([kcf[bt[0, n // 256], n % 256] if n >= 256 else np.zeros_like(kcf[0, 0])
                     for n in range(L)])
    vals = np.stack([vcf[bt[0, n // 256], n % 256] if n >= 256 else np.zeros_like(vcf[0, 0])
                     for n in range(L)])
    got = out.float().cpu().numpy()
    for j in range(2):
        vis = L - 2 + j + 1
        for h in range(8):
            s = keys[256:vis, h // 4] @ q[j, h] * 128 ** -0.5
            w = np.exp(s - s.max())
            w /= w.sum()
            ref = w @ vals[256:vis, h // 4]
            assert np.abs(got[j, h] - ref).max() <= ATTN_TOL


# ---------------------------------------------------------------- verify metadata

@pytest.mark.parametrize("num_seqs,seed", [(1, 0), (64, 1), (300, 2), (0, 3)])
def test_verify_metadata_matches_oracle(K, cuda, num_seqs, seed):
    """Device prepare_prefill for verify rows: bit-exact against the
    restatement, with empty sequences, -1 block ids, page crossings and
    padding rows (300 sequences exercise the multi-pass scan; no sequence
    at all leaves only padding rows)."""
    g = np.random.default_rng(seed)
    bs, width = 256, 12
    q = g.integers(0, 8, num_seqs).astype(np.int32)
    start = g.integers(0, bs * (width - 1) - 8, num_seqs).astype(np.int32)
    tables = g.integers(0, 5000, (num_seqs, width)).astype(np.int32)
    tables[g.random((num_seqs, width)) < 0.05] = -1
    total = int(q.sum())
    num_tokens = total + 5
    cu_q, cu_k, pos, slots = oracle.verify_metadata(start, q, tables, bs, num_tokens)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    o_cu_q = torch.full((num_seqs + 1,), -7, dtype=torch.int32, device=cuda)
    o_cu_k = torch.full((num_seqs + 1,), -7, dtype=torch.int32, device=cuda)
    o_pos = torch.full((num_tokens,), -7, dtype=torch.int64, device=cuda)
    o_slots = torch.full((num_tokens,), -7, dtype=torch.int32, device=cuda)
    K.verify_metadata(d(start), d(q), d(tables), bs, num_tokens, o_cu_q, o_cu_k, o_pos, o_slots)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o_cu_q.cpu().numpy(), cu_q)
    np.testing.assert_array_equal(o_cu_k.cpu().numpy(), cu_k)
    np.testing.assert_array_equal(o_pos.cpu().numpy(), pos)
    np.testing.assert_array_equal(o_slots.cpu().numpy(), slots)


@pytest.mark.parametrize("slot_offset", [0, 1])
@pytest.mark.parametrize("num_seqs,q_stride,seed",
                         [(1, 6, 0), (64, 6, 1), (300, 8, 2), (5, 1, 3), (0, 6, 4)])
def test_commit_metadata_matches_oracle(K, cuda, num_seqs, q_stride, seed, slot_offset):
    """Device metadata of the draft's replay of the committed tails:
    bit-exact against the restatement, from accept lengths taken straight
    from an accept-scan-shaped buffer (including out-of-range ones, which
    clamp), with -1 block ids, page crossings and padding rows, in both
    draft slot conventions (0: slot p; 1: the reference's slot p + 1)."""
    g = np.random.default_rng(seed)
    bs, width = 256, 12
    accept = g.integers(0, q_stride, num_seqs).astype(np.int32)
    accept[g.random(num_seqs) < 0.05] = q_stride + 3
    accept[g.random(num_seqs) < 0.05] = -2
    start = g.integers(0, bs * (width - 1) - 16, num_seqs).astype(np.int32)
    tables = g.integers(0, 5000, (num_seqs, width)).astype(np.int32)
    tables[g.random((num_seqs, width)) < 0.05] = -1
    t = max(num_seqs * q_stride, 5)
    argmax = g.integers(0, 151936, t).astype(np.int32)
    ref = oracle.commit_metadata(start, accept, q_stride, argmax, tables, bs, t, slot_offset)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    # the engine passes slices of the accept scan's one int32 buffer
    out = d(np.concatenate([argmax, accept, np.full(num_seqs, -9, np.int32)]))
    o_cu_q = torch.full((num_seqs + 1,), -7, dtype=torch.int32, device=cuda)
    o_cu_k = torch.full((num_seqs + 1,), -7, dtype=torch.int32, device=cuda)
    o_pos = torch.full((t,), -7, dtype=torch.int64, device=cuda)
    o_slots = torch.full((t,), -7, dtype=torch.int32, device=cuda)
    o_rows = torch.full((t,), -7, dtype=torch.int32, device=cuda)
    o_ids = torch.full((t,), -7, dtype=torch.int64, device=cuda)
    o_last = torch.full((num_seqs,), -7, dtype=torch.int64, device=cuda)
    K.commit_metadata(d(start), out[t:t + num_seqs], q_stride, out[:t], d(tables), bs, t,
                      o_cu_q, o_cu_k, o_pos, o_slots, o_rows, o_ids, o_last,
                      slot_offset=slot_offset)
    torch.cuda.synchronize()
    for got, want in zip((o_cu_q, o_cu_k, o_pos, o_slots, o_rows, o_ids, o_last), ref):
        np.testing.assert_array_equal(got.cpu().numpy(), want)


# ---------------------------------------------------------------- layer kernels + fused K2

def _qk_norm_rope_reference(qkv, positions, qw, kw, cos_sin, hq, hkv, d, eps):
    """CPU torch restatement of project_qkv's q/k RMSNorm and neox RoPE
    (models/qwen3.py:77-98, layernorm.py:70-82, rotary_embedding.py:6-48).
    Returns the rotated q, k and, for error bounds, |x1| + |x2| of each
    rotated pair (the normed inputs, repeated on both halves)."""
    t = qkv.shape[0]
    q = qkv[:, :hq * d].reshape(t, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d)

    def norm(x, w):
        if w is None:
            return x
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return xf.to(torch.bfloat16) * w

    def rope(x):
        cs = cos_sin[positions.clamp(0, cos_sin.shape[0] - 1)].unsqueeze(1)
        cos, sin = cs.chunk(2, dim=-1)
        x1, x2 = torch.chunk(x.float(), 2, dim=-1)
        mag = x1.abs() + x2.abs()
        return (torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1).to(torch.bfloat16),
                torch.cat((mag, mag), -1))

    (rq, mq), (rk, mk) = rope(norm(q, qw)), rope(norm(k, kw))
    return rq, rk, mq, mk


def _layer_case(seed, t=160, hq=16, hkv=8, d=128):
    from nanovllm_amd.layers import rope_cos_sin

    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(t, (hq + 2 * hkv) * d, generator=g) * 2.0).to(torch.bfloat16)
    positions = torch.randint(0, 4000, (t,), generator=g)
    qw = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    cos_sin = rope_cos_sin(d, 4096, 1e6, 0)
    return g, qkv, positions, qw, kw, cos_sin


@pytest.mark.parametrize("with_norm", [True, False])
def test_qk_norm_rope_matches_reference_formulas(K, cuda, with_norm):
    """The kernel's fp32 mean runs in a different summation order than
    torch's, so a normed element may round to the neighbouring bf16 value;
    the rotation then carries that one-ulp input difference (bounded by
    2^-7 (|x1| + |x2|) of the pair) plus one ulp of its own rounding.
    Nearly every element is identical."""
    hq, hkv, d = 16, 8, 128
    _, qkv, pos, qw, kw, cos_sin = _layer_case(31)
    qw, kw = (qw, kw) if with_norm else (None, None)
    q, k = K.qk_norm_rope(qkv.to(cuda), pos.to(cuda), None if qw is None else qw.to(cuda),
                          None if kw is None else kw.to(cuda), cos_sin, hq, hkv, d, 1e-6)
    rq, rk, mq, mk = _qk_norm_rope_reference(qkv, pos, qw, kw, cos_sin.cpu(), hq, hkv, d, 1e-6)
    for got, ref, mag in ((q.cpu(), rq, mq), (k.cpu(), rk, mk)):
        diff = (got.float() - ref.float()).abs()
        bound = (ref.float().abs() + (mag if with_norm else 0.0)) * 2.0 ** -7 * 1.01
        assert bool((diff <= bound + 1e-30).all()), float((diff - bound).max())
        assert float((got == ref).float().mean()) > 0.99


@pytest.mark.parametrize("layout", ["token_major", "head_major"])
@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("with_norm", [True, False])
def test_qk_norm_rope_store_matches_separate_kernels(K, cuda, layout, fp8, with_norm):
    """The fused launch leaves q and both caches bit-identical to
    qk_norm_rope followed by store_kvcache (negative and out-of-range slots
    skipped, FP8 scales applied)."""
    hq, hkv, d, nb, bs = 16, 8, 128, 12, 256
    g, qkv, pos, qw, kw, cos_sin = _layer_case(33)
    t = qkv.shape[0]
    slots = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    slots[::7] = -1
    slots[3] = nb * bs + 5
    cdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    init = torch.randn(nb, bs, hkv, d, generator=g).to(cdt)

    def cache():
        if layout == "head_major":
            return init.permute(0, 2, 1, 3).contiguous().to(cuda).permute(0, 2, 1, 3)
        return init.clone().to(cuda)

    ks = torch.tensor([0.75], device=cuda) if fp8 else None
    vs = torch.tensor([1.5], device=cuda) if fp8 else None
    dq, dpos, dslots = qkv.to(cuda), pos.to(cuda), slots.to(cuda)
    dqw = qw.to(cuda) if with_norm else None
    dkw = kw.to(cuda) if with_norm else None
    kc1, vc1, kc2, vc2 = cache(), cache(), cache(), cache()
    q1, k1 = K.qk_norm_rope(dq, dpos, dqw, dkw, cos_sin, hq, hkv, d, 1e-6)
    K.store_kvcache(k1, dq[:, (hq + hkv) * d:].view(t, hkv, d), kc1, vc1, dslots, ks, vs)
    q2 = K.qk_norm_rope_store(dq, dpos, dqw, dkw, cos_sin, hq, hkv, d, 1e-6, kc2, vc2, dslots,
                              ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.int16).cpu(), q2.view(torch.int16).cpu())
    for a, b in ((kc1, kc2), (vc1, vc2)):
        np.testing.assert_array_equal(bits(a.contiguous().cpu()), bits(b.contiguous().cpu()))
    # the rows with a valid slot did change
    changed = bits(kc2.contiguous().cpu()) != bits(init)
    assert changed.any()


@pytest.mark.parametrize("inter", [1000, 4104])
def test_silu_mul_vector_path_matches_scalar_and_reference(K, cuda, inter):
    """16-byte vector path == element path (bit-exact); both within one bf16
    ulp of torch's bf16(bf16(silu(a)) * b) (activation.py:11-14), whose exp
    may round differently from the device's.  4104 = 513 vectors a row: the
    row's last block holds a single vector."""
    g = torch.Generator().manual_seed(41)
    rows = 40
    full = (torch.randn(rows, 2 * inter + 1, generator=g) * 3).to(torch.bfloat16).to(cuda)
    x_vec = full[:, :2 * inter].contiguous()           # row stride 2000: vector path
    x_scalar = full[:, :2 * inter]                      # row stride 2001: element path
    assert torch.equal(x_vec, x_scalar)
    y_vec, y_scalar = K.silu_mul(x_vec), K.silu_mul(x_scalar)
    torch.cuda.synchronize()
    assert torch.equal(y_vec.view(torch.int16), y_scalar.view(torch.int16))
    a, b = x_vec.cpu()[:, :inter], x_vec.cpu()[:, inter:]
    ref = torch.nn.functional.silu(a) * b
    diff = (y_vec.cpu().float() - ref.float()).abs()
    assert bool((diff <= ref.float().abs() * 2.0 ** -7 * 1.01 + 1e-30).all())
    assert float((y_vec.cpu() == ref).float().mean()) > 0.99


@pytest.mark.parametrize("h", [4096, 5120, 8192, 12288])
@pytest.mark.parametrize("add", [False, True])
def test_rms_norm_matches_reference_formulas(K, cuda, add, h):
    """rms_forward / add_rms_forward (layernorm.py:70-107): the fp32 (sum) row
    is normalised, rounded to bf16, multiplied by the bf16 weight; the new
    residual is bf16(x + residual) exactly.  Rows of up to 8192 stay in
    registers between the reduction and the normalisation, 12288 takes the
    two-pass loop."""
    g = torch.Generator().manual_seed(43)
    rows = 96
    x = (torch.randn(rows, h, generator=g) * 2).to(torch.bfloat16)
    r = torch.randn(rows, h, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    s = x.float() + r.float() if add else x.float()
    ref = (s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * w
    if add:
        out, res = K.add_rms_norm(x.to(cuda), r.to(cuda), w.to(cuda), 1e-6)
        assert torch.equal(res.cpu().view(torch.int16), s.to(torch.bfloat16).view(torch.int16))
    else:
        out = K.rms_norm(x.to(cuda), w.to(cuda), 1e-6)
    got = out.cpu()
    diff = (got.float() - ref.float()).abs()
    assert bool((diff <= ref.float().abs() * 2.0 ** -7 * 1.01 + 1e-30).all())
    assert float((got == ref).float().mean()) > 0.99


def test_add_then_rms_norm_equals_add_followed_by_rms_norm(K, cuda):
    """The EAGLE3 draft's fused residual add + norm is bit-identical to a bf16
    tensor add followed by rms_norm (eagle3.py:141-146), also with a strided
    residual (a half of the attention input) and on the element path."""
    g = torch.Generator().manual_seed(45)
    for rows, h in ((64, 4096), (7, 1000)):
        x = (torch.randn(rows, h, generator=g) * 2).to(torch.bfloat16).to(cuda)
        wide = torch.randn(rows, 2 * h, generator=g).to(torch.bfloat16).to(cuda)
        r = wide[:, h:]
        w = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16).to(cuda)
        out, total = K.add_then_rms_norm(x, r, w, 1e-6)
        ref_total = x + r
        ref_out = K.rms_norm(ref_total, w, 1e-6)
        torch.cuda.synchronize()
        assert torch.equal(total.view(torch.int16), ref_total.view(torch.int16))
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        # and it is not the fp32-sum variant on these inputs
        out32, _ = K.add_rms_norm(x, r, w, 1e-6)
        assert not torch.equal(out32.view(torch.int16), out.view(torch.int16))


def test_rms_norm_into_strided_halves(K, cuda):
    """rms_norm writing into the halves of a [rows, 2H] buffer equals the
    concatenation of two separate results (the draft's attention input)."""
    g = torch.Generator().manual_seed(47)
    a = torch.randn(64, 4096, generator=g).to(torch.bfloat16).to(cuda)
    b = torch.randn(64, 4096, generator=g).to(torch.bfloat16).to(cuda)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(cuda)
    both = torch.empty(64, 8192, dtype=torch.bfloat16, device=cuda)
    K.rms_norm(a, w, 1e-6, out=both[:, :4096])
    K.rms_norm(b, w, 1e-6, out=both[:, 4096:])
    ref = torch.cat((K.rms_norm(a, w, 1e-6), K.rms_norm(b, w, 1e-6)), -1)
    torch.cuda.synchronize()
    assert torch.equal(both.view(torch.int16), ref.view(torch.int16))


# ---------------------------------------------------------------- K1 at full BASELINE sizes

FULL_CASES = {
    # BASELINE config 3's verify: B64, q6, 32/8 heads, L ~ U[256, 2304]: 24-row
    # tiles in paired mode (four waves per whole sequence, grid rows past
    # CUs / Hkv taking the sequences from the last one backwards)
    "config3": dict(seed=2, batch=64, q_len=6, ctx_lo=256, ctx_hi=2304, hq=32, hkv=8),
    # paired mode with part of the CUs holding one segment (320 segments)
    "config3_b40": dict(seed=12, batch=40, q_len=6, ctx_lo=256, ctx_hi=2304, hq=32, hkv=8),
    # FP8 pages, B128, q5, 16/8 heads, L ~ U[4096, 16384]
    "config4_fp8": dict(seed=3, batch=128, q_len=5, ctx_lo=4096, ctx_hi=16384, hq=16, hkv=8,
                        fp8=True),
    # B128, q8, 64/8 heads, L ~ U[2048, 8192], 30% shared prefix pages
    "config5": dict(seed=4, batch=128, q_len=8, ctx_lo=2048, ctx_hi=8192, hq=64, hkv=8,
                    shared_frac=0.3),
}


@pytest.mark.parametrize("name", list(FULL_CASES))
def test_full_size_verify_matches_decode_rows(K, cuda, name):
    """At the BASELINE configs' full sizes (too large for the CPU oracle):
    every verify row equals the decode entry's row with context length
    L_i - q_i + j + 1 on the same pages (the reference's config-4 comparator:
    a verify row expanded into a paged decode row, attention.py:249-293),
    although the two launches decompose the keys differently (stream ranges
    or 3072-key splits with a combine, against per-row splits)."""
    from helpers import device_paged_case

    c = device_paged_case(cuda, **FULL_CASES[name])
    q_len, lens = c["q_len"], c["lens"]
    one = torch.ones(1, device=cuda) if FULL_CASES[name].get("fp8") else None
    out = K.paged_attention_varlen(c["q"], c["k_cache"], c["v_cache"], c["cu_q"], c["cu_k"],
                                   q_len, c["max_k"], 128 ** -0.5, c["block_tables"],
                                   k_scale=one, v_scale=one)
    ctx = torch.tensor([L - q_len + j + 1 for L in lens for j in range(q_len)],
                       dtype=torch.int32, device=cuda)
    rows_bt = c["block_tables"].repeat_interleave(q_len, dim=0).contiguous()
    dec = K.paged_attention_decode(c["q"], c["k_cache"], c["v_cache"], ctx, rows_bt,
                                   128 ** -0.5, max_seqlen_k=c["max_k"], k_scale=one,
                                   v_scale=one)
    torch.cuda.synchronize()
    err = (out.float() - dec.float()).abs().max().item()
    scale = dec.float().abs().max().item()
    assert bool(torch.isfinite(out.float()).all()) and scale > 1e-3, (name, scale)
    # the north star's 2e-2, and a few bf16 ulps of the output's own scale
    assert err <= min(ATTN_TOL, 1e-2 * scale), (name, err, scale)


@pytest.mark.parametrize("name", list(FULL_CASES))
def test_full_size_verify_constant_values(K, cuda, name):
    """Softmax weights sum to one: with every V row of kv head h equal to
    one vector c_h, every output row of the heads sharing it is c_h, across
    all splits, stream ranges and the combine, at full size."""
    from helpers import device_paged_case

    case = FULL_CASES[name]
    c = device_paged_case(cuda, **case)
    hkv = case["hkv"]
    g = torch.Generator(device=cuda).manual_seed(77)
    cvec = (torch.rand(hkv, 128, generator=g, device=cuda) - 0.5).to(torch.bfloat16)
    if case.get("fp8"):
        cvec = cvec.float().to(torch.float8_e4m3fn)
    # pages [blocks, Hkv, 2, block_size, D]: V is index 1 of dim 2
    c["pages"][:, :, 1] = cvec[None, :, None, :].to(c["pages"].dtype)
    one = torch.ones(1, device=cuda) if case.get("fp8") else None
    out = K.paged_attention_varlen(c["q"], c["k_cache"], c["v_cache"], c["cu_q"], c["cu_k"],
                                   c["q_len"], c["max_k"], 128 ** -0.5, c["block_tables"],
                                   k_scale=one, v_scale=one)
    torch.cuda.synchronize()
    group = case["hq"] // hkv
    want = cvec.float().repeat_interleave(group, dim=0)          # [Hq, D]
    err = (out.float() - want[None]).abs().max().item()
    assert err <= 1e-2 * want.abs().max().item() + 1e-6, (name, err)


def _sample_rows(c, picks):
    """Host copies of the pages, query rows and output rows of the sampled
    sequences of a device_paged_case, re-addressed through a compact block
    table (sequence n's blocks become ids off_n .. off_n + blocks - 1)."""
    pages, bt, lens, q_len = c["pages"], c["block_tables"], c["lens"], c["q_len"]
    bs = pages.shape[3]
    ks, vs, tables, off = [], [], [], 0
    for i in picks:
        n = -(-lens[i] // bs)
        pg = pages[bt[i, :n].long()].cpu()                # [n, Hkv, 2, bs, D]
        ks.append(pg[:, :, 0].permute(0, 2, 1, 3))        # [n, bs, Hkv, D]
        vs.append(pg[:, :, 1].permute(0, 2, 1, 3))
        tables.append(list(range(off, off + n)))
        off += n
    width = max(len(t) for t in tables)
    sub_bt = np.full((len(picks), width), -1, np.int32)
    for r, t in enumerate(tables):
        sub_bt[r, :len(t)] = t
    rows = torch.tensor([i * q_len + j for i in picks for j in range(q_len)])
    q = c["q"].index_select(0, rows.to(c["q"].device)).cpu()
    return (bits(torch.cat(ks).contiguous()), bits(torch.cat(vs).contiguous()), sub_bt, rows,
            bits(q), np.array([lens[i] for i in picks], np.int32))


def _picks(c, count, seed):
    """The longest and the shortest sequence plus seeded random others."""
    lens = np.array(c["lens"])
    rng = np.random.default_rng(seed)
    picks = {int(lens.argmax()), int(lens.argmin())}
    while len(picks) < count:
        picks.add(int(rng.integers(len(lens))))
    return sorted(picks)


@pytest.mark.parametrize("name", list(FULL_CASES))
def test_full_size_verify_matches_oracle_on_sampled_sequences(K, cuda, name):
    """At the BASELINE configs' full sizes the whole batch runs on the GPU in
    one launch (config 3: 24-row tiles in paired mode, 64 and 40 sequences;
    config 4: FP8 pages, stream ranges over 128 sequences of
    4096-16384 keys; config 5: 64-row tiles, splits of three quarters of
    the longest sequence (6144 keys) and the combine, the first 30% of
    every sequence's blocks shared), and the
    rows of 8 sampled sequences -- the longest and the shortest among them
    -- are held to the CPU oracle on the same pages: the textbook attention
    within 2e-2 (the north star's bound) and, for FP8, the restated
    reference FP8 decode kernel (attention.py:85-182) within 2e-3 with each
    verify row expanded into a decode row of context L_i - q_i + j + 1."""
    from helpers import device_paged_case

    case = FULL_CASES[name]
    c = device_paged_case(cuda, **case)
    fp8 = case.get("fp8", False)
    one = torch.ones(1, device=cuda) if fp8 else None
    out = K.paged_attention_varlen(c["q"], c["k_cache"], c["v_cache"], c["cu_q"], c["cu_k"],
                                   c["q_len"], c["max_k"], 128 ** -0.5, c["block_tables"],
                                   k_scale=one, v_scale=one)
    torch.cuda.synchronize()
    picks = _picks(c, 8, seed=5)
    if name == "config5":
        # at least one sampled sequence is split (and combined)
        assert max(c["lens"][i] for i in picks) > 6144
    kb, vb, sub_bt, rows, qb, lens = _sample_rows(c, picks)
    q_len = c["q_len"]
    cu = np.arange(0, len(picks) * q_len + 1, q_len, dtype=np.int32)
    got = out.index_select(0, rows.to(cuda)).float().cpu().numpy()
    ref = oracle.paged_attention(qb, kb, vb, cu, lens, sub_bt, 128 ** -0.5)
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL, (name, err, picks)
    if fp8:
        ctx = np.array([L - q_len + j + 1 for L in lens for j in range(q_len)], np.int32)
        dec = oracle.fp8_paged_decode(qb, kb, vb, ctx, np.repeat(sub_bt, q_len, axis=0),
                                      128 ** -0.5)
        err_dec = np.abs(got - dec).max()
        assert err_dec <= FP8_TOL, (name, err_dec, picks)


@pytest.mark.parametrize("name,kw,clip_to", [
    # fixed decomposition, 40-row tiles (NT 4) with splits and the combine
    ("gqa8_fixed", dict(seed=12, batch=6, q_len=[8, 3, 8, 5, 8, 1], ctx_lo=3500, ctx_hi=8000,
                        hq=64, hkv=8), 5),
    # fixed decomposition, eight waves per split (16-row tiles)
    ("gqa4_shared", dict(seed=13, batch=5, q_len=[6, 6, 2, 6, 4], ctx_lo=300, ctx_hi=5000,
                         hq=32, hkv=8), 4),
    # FP8 stream decomposition
    ("fp8_stream", dict(seed=14, batch=6, q_len=[5, 2, 5, 5, 3, 5], ctx_lo=300, ctx_hi=5000,
                        hq=16, hkv=8, fp8=True), 3),
])
def test_rows_past_max_seqlen_q_are_cleared(K, cuda, name, kw, clip_to):
    """A max_seqlen_q below a sequence's query count clips it: its rows past
    the bound come back as zeros, its kept rows keep their exact causal
    windows, and the combine does not merge the stale split counts an
    earlier call left in the shared workspace for those rows (the first
    call below runs the same batch unclipped and leaves counts > 1)."""
    kw = dict(kw)
    fp8 = kw.pop("fp8", False)
    case = paged_case(**kw)
    kc, vc = case["k_cache"], case["v_cache"]
    if fp8:
        kc, vc = kc.float().to(torch.float8_e4m3fn), vc.float().to(torch.float8_e4m3fn)
    dkc, dvc = kc.to(cuda), vc.to(cuda)
    one = torch.ones(1, device=cuda) if fp8 else None
    args = (dkc, dvc, case["cu_q"].to(cuda), case["cu_k"].to(cuda))
    q = case["q"].to(cuda)
    max_k = int(case["lens"].max())
    full = K.paged_attention_varlen(q, *args, max(case["q_lens"]), max_k, 128 ** -0.5,
                                    case["block_tables"].to(cuda), k_scale=one, v_scale=one)
    out = torch.full_like(q, 7.0)
    K.paged_attention_varlen(q, *args, clip_to, max_k, 128 ** -0.5, case["block_tables"].to(cuda),
                             k_scale=one, v_scale=one, out=out)
    torch.cuda.synchronize()
    got, full = out.float().cpu(), full.float().cpu()
    cu = case["cu_q"].tolist()
    kept_rows, kept_q, kept_lens = [], [], []
    for i, (qn, L) in enumerate(zip(case["q_lens"], case["lens"].tolist())):
        keep = min(qn, clip_to)
        kept_rows += range(cu[i], cu[i] + keep)
        kept_q.append(keep)
        kept_lens.append(L - (qn - keep))
        assert bool((got[cu[i] + keep:cu[i + 1]] == 0).all()), (name, i)
    kept = torch.tensor(kept_rows)
    # kept rows: the same values as the unclipped call (to the last bit is
    # not promised: the split decomposition follows max_seqlen_q) ...
    assert (got[kept] - full[kept]).abs().max().item() <= 2e-3, name
    # ... and the oracle of the kept rows with their unclipped windows
    ref = oracle.paged_attention(bits(case["q"][kept]), bits(kc), bits(vc),
                                 np.array([0] + np.cumsum(kept_q).tolist(), np.int32),
                                 np.array(kept_lens, np.int32), case["block_tables"].numpy(),
                                 128 ** -0.5)
    assert np.abs(got[kept].numpy() - ref).max() <= ATTN_TOL, name


def test_wrappers_refuse_bounds_below_host_lengths(K, cuda):
    """Host-known lengths (CPU tensors or lists) let the wrappers refuse a
    max_seqlen below them before any launch; with a sufficient bound the
    host arguments give the same result as device tensors."""
    case = paged_case(seed=15, batch=4, q_len=[3, 5, 2, 5], ctx_lo=50, ctx_hi=900, hq=16, hkv=8)
    kc, vc = case["k_cache"].to(cuda), case["v_cache"].to(cuda)
    q, bt = case["q"].to(cuda), case["block_tables"].to(cuda)
    max_k = int(case["lens"].max())
    with pytest.raises(ValueError, match="max_seqlen_q=4"):
        K.paged_attention_varlen(q, kc, vc, case["cu_q"], case["cu_k"], 4, max_k, 0.1, bt)
    with pytest.raises(ValueError, match="max_seqlen_k"):
        K.paged_attention_varlen(q, kc, vc, case["cu_q"].tolist(), case["cu_k"], 5, max_k - 1,
                                 0.1, bt)
    with pytest.raises(ValueError, match="max_seqlen_k"):
        K.paged_attention_decode(q[:4], kc, vc, case["lens"], bt, 0.1, max_seqlen_k=max_k - 1)
    host = K.paged_attention_varlen(q, kc, vc, case["cu_q"], case["cu_k"], 5, max_k, 0.1, bt)
    dev = K.paged_attention_varlen(q, kc, vc, case["cu_q"].to(cuda), case["cu_k"].to(cuda), 5,
                                   max_k, 0.1, bt)
    torch.cuda.synchronize()
    assert torch.equal(host.view(torch.int16), dev.view(torch.int16))


def test_verify_input_ids_from_proposals(K, cuda):
    """nva_verify_input_ids against the reference's own route to the verify
    input: each sequence's proposals appended to its tokens
    (llm_engine.py:129-141), then its last k + 1 tokens read from
    num_computed_tokens = len - 1 (model_runner.py:770-774); rows in the
    longest-first verify order, padding rows 0, and compose = 0 leaving the
    host's ids in place."""
    g = torch.Generator().manual_seed(53)
    bs, b, k = 16, 11, 5
    q = k + 1
    seqs = [torch.randint(0, 151936, (int(n),), generator=g).tolist()
            for n in torch.randint(1, 40, (b,), generator=g)]
    props = torch.randint(0, 151936, (k, bs), generator=g)
    order = sorted(range(b), key=lambda i: -len(seqs[i]))
    want = []
    for i in order:
        tokens = seqs[i] + props[:, i].tolist()
        start = len(seqs[i]) - 1
        want += tokens[start:start + q]
    want += [0] * ((bs - b) * q)
    compose = torch.ones(1, dtype=torch.int32, device=cuda)
    last = torch.tensor([seqs[i][-1] for i in order] + [0] * (bs - b), dtype=torch.int32)
    cols = torch.tensor(order + [-1] * (bs - b - 1) + [bs], dtype=torch.int32)  # bs: out of range
    ids = torch.full((bs * q,), 7, dtype=torch.int64, device=cuda)
    K.verify_input_ids(compose, last.to(cuda), cols.to(cuda), props.to(cuda), q, ids)
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == want
    compose.zero_()
    host = torch.arange(bs * q, dtype=torch.int64, device=cuda)
    K.verify_input_ids(compose, last.to(cuda), cols.to(cuda), props.to(cuda), q, host)
    torch.cuda.synchronize()
    assert torch.equal(host.cpu(), torch.arange(bs * q))


def test_draft_metadata_after_verify(K, cuda):
    """nva_draft_metadata: each column's length after the verified step is
    lens + accept[verify_row] + 1 and its draft steps sit at the positions
    after it, slots through its block-table row (the host loop of
    model_runner.py:1087-1096 restated per element); padding columns,
    positions past the table and negative block ids give slot -1."""
    g = torch.Generator().manual_seed(51)
    bs, b, steps, bsz, mb = 16, 11, 4, 32, 6
    lens = torch.randint(1, bsz * mb - 12, (bs,), generator=g)
    lens[b:] = 0
    lens[3] = bsz * mb - 3                       # its later steps run past the table
    vrow = torch.randperm(bs, generator=g)
    accept = torch.randint(0, 5, (bs,), generator=g).to(torch.int32)
    bt = torch.randint(0, 500, (bs, mb), generator=g).to(torch.int32)
    bt[5, 2] = -1                                # a negative block id
    bt[b:] = -1
    pos = torch.zeros(steps, bs, dtype=torch.int64, device=cuda)
    slots = torch.zeros(steps, bs, dtype=torch.int32, device=cuda)
    ctx = torch.zeros(steps, bs, dtype=torch.int32, device=cuda)
    K.draft_metadata(lens.to(cuda), vrow.to(cuda), accept.to(cuda), bs, bt.to(cuda), bsz, pos,
                     slots, ctx)
    torch.cuda.synchronize()
    want_pos = torch.zeros(steps, bs, dtype=torch.int64)
    want_slot = torch.full((steps, bs), -1, dtype=torch.int32)
    for i in range(bs):
        new_len = int(lens[i]) + int(accept[int(vrow[i])]) + 1
        for s in range(steps):
            p = new_len - 1 + s
            want_pos[s, i] = p
            blk = p // bsz
            if blk < mb and int(bt[i, blk]) >= 0:
                want_slot[s, i] = int(bt[i, blk]) * bsz + p % bsz
    assert torch.equal(pos.cpu(), want_pos)
    assert torch.equal(slots.cpu(), want_slot)
    assert torch.equal(ctx.cpu(), (want_pos + 1).to(torch.int32))
    assert (want_slot[:, 3] == -1).any() and (want_slot[:, b:] == -1).all()
    # both draft slot conventions against the oracle's restatement (offset 1
    # is the reference's slot len + step, context len + step + 1)
    for off in (0, 1):
        K.draft_metadata(lens.to(cuda), vrow.to(cuda), accept.to(cuda), b, bt.to(cuda), bsz, pos,
                         slots, ctx, slot_offset=off)
        torch.cuda.synchronize()
        opos, oslots, octx = oracle.draft_metadata(lens.numpy(), vrow.numpy(), accept.numpy(), b,
                                                   bs, steps, bt.numpy(), bsz, off)
        np.testing.assert_array_equal(pos.cpu().numpy(), opos)
        np.testing.assert_array_equal(slots.cpu().numpy(), oslots)
        np.testing.assert_array_equal(ctx.cpu().numpy(), octx)
