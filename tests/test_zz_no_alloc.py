"""The allocation-free argmax + acceptance entry point
(``nva_argmax_accept_static``) against the workspace entry point
``nva_argmax_accept``, bit for bit, through the C ABI.

Three calls in a row, each smaller than the one before: a batch near the
static array's limit (6553 rows of a 151936-token vocabulary, 65530 chunk
keys), then BASELINE config 3's verify rows [64 x 6], then config 1's [8 x 5].
The static array keeps the previous call's keys, so a merge that read a key
the current call did not write would show up in the smaller calls.  One row
more than the limit is refused on the host with ValueError before anything
is launched.
"""
import numpy as np
import pytest
import torch

from helpers import acceptance_logits
from oracle import oracle

pytestmark = pytest.mark.gpu

VOCAB = 151936
LIMIT_ROWS = 65536 // -(-VOCAB // 16384)          # 6553 rows of 10 chunks


@pytest.fixture(scope="module")
def K(cuda):
    from nanovllm_amd import kernels

    return kernels


def _both(K, logits, cu_q, ids):
    t, b = logits.shape[0], cu_q.numel() - 1
    out_ws = torch.full((t + 2 * b,), -7, dtype=torch.int32, device=logits.device)
    out_st = torch.full((t + 2 * b,), -7, dtype=torch.int32, device=logits.device)
    K.argmax_accept(logits, cu_q, ids, out=out_ws)
    K.argmax_accept_static(logits, cu_q, ids, out_st)
    torch.cuda.synchronize()
    return out_ws.cpu().numpy(), out_st.cpu().numpy()


def _near_limit_batch(cuda, rows):
    """Ragged verify batch of ``rows`` rows (q_i in 1..8) generated on the
    device; about half the proposals equal the target's argmax so the scan
    accepts prefixes of every length."""
    g = torch.Generator(device=cuda).manual_seed(31)
    logits = torch.randn(rows, VOCAB, generator=g, device=cuda).to(torch.bfloat16)
    gh = torch.Generator().manual_seed(31)
    qs = []
    while sum(qs) < rows:
        qs.append(min(int(torch.randint(1, 9, (1,), generator=gh)), rows - sum(qs)))
    cu_q = torch.tensor([0] + np.cumsum(qs).tolist(), dtype=torch.int32, device=cuda)
    am = logits.argmax(-1)
    ids = torch.randint(0, VOCAB, (rows,), generator=g, device=cuda)
    take = torch.rand(rows, generator=g, device=cuda) < 0.8
    ids[1:] = torch.where(take[1:], am[:-1], ids[1:])
    return logits, cu_q, ids.contiguous()


def test_static_entry_equals_workspace_entry_on_shrinking_calls(K, cuda):
    big, cu_big, ids_big = _near_limit_batch(cuda, LIMIT_ROWS + 1)
    # one row past the limit: refused on the host, nothing launched
    b_over = cu_big.numel() - 1
    out_over = torch.empty(big.shape[0] + 2 * b_over, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="static scratch capacity"):
        K.argmax_accept_static(big, cu_big, ids_big, out_over)
    # call 1: exactly at the limit's row count (a sequence boundary may cut
    # the last sequence short, which is fine: cu_q ends at LIMIT_ROWS)
    cu1 = cu_big.clone()
    cu1[cu1 > LIMIT_ROWS] = LIMIT_ROWS
    cu1 = torch.unique_consecutive(cu1)
    logits1, ids1 = big[:LIMIT_ROWS], ids_big[:LIMIT_ROWS].contiguous()
    ws, st = _both(K, logits1, cu1, ids1)
    np.testing.assert_array_equal(st, ws)
    b1 = cu1.numel() - 1
    acc1 = st[LIMIT_ROWS:LIMIT_ROWS + b1]
    assert acc1.max() >= 4 and (acc1 == 0).any(), "the batch must exercise the scan"
    host = logits1.cpu().view(torch.int16).numpy().view(np.uint16)
    del big, logits1
    np.testing.assert_array_equal(st[:LIMIT_ROWS], oracle.argmax_bf16(host))
    # calls 2 and 3: config 3's and config 1's verify batches, each smaller
    for batch, k, seed in ((64, 5, 2), (8, 4, 0)):
        logits, cu_q, ids, _ = acceptance_logits(batch, k, VOCAB, 0.7, seed)
        ws, st = _both(K, logits.to(cuda), cu_q.to(cuda), ids.to(cuda))
        np.testing.assert_array_equal(st, ws)
        t = logits.shape[0]
        ref_am = oracle.argmax_bf16(logits.view(torch.int16).numpy().view(np.uint16))
        ref_acc, ref_bonus = oracle.accept(cu_q.numpy(), ref_am, ids.numpy())
        np.testing.assert_array_equal(st[:t], ref_am)
        np.testing.assert_array_equal(st[t:t + batch], ref_acc)
        np.testing.assert_array_equal(st[t + batch:], ref_bonus)


def test_static_entry_under_graph_capture_and_replay(K, cuda):
    """One ordinary call (the per-device address lookup happens there), then
    the entry point recorded into a HIP graph and replayed: every replay,
    with new logits copied into the captured input between replays and the
    host's own eager work in between, equals the workspace entry point bit
    for bit."""
    batch, k = 64, 5
    logits, cu_q, ids, _ = acceptance_logits(batch, k, VOCAB, 0.7, 11)
    t = logits.shape[0]
    x = logits.to(cuda)
    cu_d, ids_d = cu_q.to(cuda), ids.to(cuda)
    out = torch.full((t + 2 * batch,), -7, dtype=torch.int32, device=cuda)
    K.argmax_accept_static(x, cu_d, ids_d, out)          # the warm-up call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.argmax_accept_static(x, cu_d, ids_d, out)
    torch.cuda.synchronize()
    for rep in range(4):
        fresh, _, _, _ = acceptance_logits(batch, k, VOCAB, 0.7, 100 + rep)
        x.copy_(fresh.to(cuda))
        out.fill_(-9)
        g.replay()
        want = torch.empty_like(out)
        K.argmax_accept(x, cu_d, ids_d, out=want)        # eager, between replays
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), want.cpu().numpy())
        assert (out[t:t + batch] >= 0).all()
