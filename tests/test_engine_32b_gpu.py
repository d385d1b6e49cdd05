"""End-to-end greedy equality at BASELINE config 5's geometry: Qwen3-32B
(64 layers, hidden 5120, 64 q / 8 kv heads (GQA group 8), MLP 25600,
vocabulary 151936, random weights), an EAGLE3 draft with k = 7 (8 verify
rows per sequence, so 64-row attention tiles per kv head), contexts drawn
from U[2048, 8192], pages handed out in a shuffled order (fragmented block
tables), through the graphed, pipelined engine.  Batch 16 instead of the
config's 128 keeps the test within its budget; the attention tiles, the
split-KV path of the long sequences and every kernel shape per sequence are
the config's.  The rule, its tolerance (measured from the non-speculative
engine in the same run) and the forced drafts are described in
tests/greedy_e2e.py."""
import pytest
import torch

from greedy_e2e import run
from nanovllm_amd import LLM
from nanovllm_amd.synthetic import default_aux_layers, write_eagle3_config, write_qwen3_config

pytestmark = pytest.mark.gpu

BATCH = 16
K_SPEC = 7
MAX_TOKENS = 96
PROMPT_RANGE = (2048, 8192)


@pytest.fixture(scope="module")
def dirs(tmp_path_factory):
    root = tmp_path_factory.mktemp("ckpt32b")
    aux = default_aux_layers("qwen3-32b")
    return (write_qwen3_config(str(root / "target"), "qwen3-32b"),
            write_eagle3_config(str(root / "draft"), "qwen3-32b", aux_layers=aux), aux)


def test_config5_geometry_spec_equals_target_greedy(dirs):
    target, draft, aux = dirs
    pages = BATCH * (-(-(PROMPT_RANGE[1] + MAX_TOKENS + 2 * K_SPEC + 2) // 256)) + 40

    def make_llm(spec):
        kw = dict(load_format="dummy", seed=0, max_model_len=PROMPT_RANGE[1] + MAX_TOKENS + 16,
                  num_kvcache_blocks=pages, enforce_eager=False, max_num_batched_tokens=16384,
                  max_num_seqs=BATCH, enable_prefill_batching=True)
        if spec:
            kw["speculative_config"] = {"method": "eagle3", "model": draft,
                                        "num_speculative_tokens": K_SPEC,
                                        "aux_hidden_state_layers": aux}
        return LLM(target, **kw)

    g = torch.Generator().manual_seed(4)
    lens = torch.randint(PROMPT_RANGE[0], PROMPT_RANGE[1] + 1, (BATCH,), generator=g).tolist()
    prompts = [torch.randint(0, 151936, (n,), generator=g).tolist() for n in lens]
    summary = run(make_llm, prompts, K_SPEC, MAX_TOKENS, "config5", page_seed=40)
    # the speculative steps verified 64-row tiles (8 rows x group 8) on every
    # sequence; at this batch a tile's keys are cut into 3072-key splits, so
    # most sequences also ran the split-KV path and its combine
    assert sum(n > 3072 for n in lens) > BATCH // 2, lens
    assert summary["stats"]["steps"] > 0
