"""End-to-end greedy equality at BASELINE config 3's geometry: Qwen3-8B
(36 layers, hidden 4096, 32 q / 8 kv heads, MLP 12288, vocabulary 151936,
random weights), an EAGLE3 draft on aux layers 2/18/33, k = 5, batch 64,
prompts drawn from U[256, 2048], 256 output tokens per sequence, through
the graphed, pipelined engine.  The rule, its tolerance (measured from the
non-speculative engine in the same run) and the forced drafts are described
in tests/greedy_e2e.py."""
import pytest
import torch

from greedy_e2e import run
from nanovllm_amd import LLM
from nanovllm_amd.synthetic import write_eagle3_config, write_qwen3_config

pytestmark = pytest.mark.gpu

BATCH = 64
K_SPEC = 5
MAX_TOKENS = 256


@pytest.fixture(scope="module")
def dirs(tmp_path_factory):
    root = tmp_path_factory.mktemp("ckpt8b")
    return (write_qwen3_config(str(root / "target"), "qwen3-8b"),
            write_eagle3_config(str(root / "draft"), "qwen3-8b"))


def test_config3_geometry_spec_equals_target_greedy(dirs):
    target, draft = dirs

    def make_llm(spec):
        # the whole batch prefills in one step, so every decode step holds
        # all 64 sequences (the bench's shape)
        kw = dict(load_format="dummy", seed=0, max_model_len=2304, num_kvcache_blocks=720,
                  enforce_eager=False, max_num_batched_tokens=131072, max_num_seqs=BATCH,
                  enable_prefill_batching=True)
        if spec:
            kw["speculative_config"] = {"method": "eagle3", "model": draft,
                                        "num_speculative_tokens": K_SPEC}
        return LLM(target, **kw)

    g = torch.Generator().manual_seed(2)
    lens = torch.randint(256, 2049, (BATCH,), generator=g).tolist()
    prompts = [torch.randint(0, 151936, (n,), generator=g).tolist() for n in lens]
    run(make_llm, prompts, K_SPEC, MAX_TOKENS, "config3")
