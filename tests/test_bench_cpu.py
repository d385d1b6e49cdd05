"""bench.py's host-side rules (no GPU): the recorded HBM-traffic constant is
quoted only for the workload and the attention-kernel source it was read
on."""
import argparse

import bench


def _default_args(**over):
    kw = dict(bench.PMC_WORKLOAD)
    kw.update(over)
    return argparse.Namespace(**kw)


def test_traffic_constant_follows_the_kernel_source(monkeypatch):
    monkeypatch.setattr(bench, "PMC_ATTENTION_SOURCE", bench.attention_source_hash())
    assert bench.pmc_traffic_reason(_default_args()) is None
    assert bench.pmc_traffic_bytes(_default_args()) == bench.PMC_TRAFFIC_BYTES
    # another workload, or another kernel source: no figure, and the reason
    assert "default workload" in bench.pmc_traffic_reason(_default_args(batch=32))
    assert bench.pmc_traffic_bytes(_default_args(kv_layout="token_major")) is None
    monkeypatch.setattr(bench, "PMC_ATTENTION_SOURCE", "0" * 16)
    assert "source" in bench.pmc_traffic_reason(_default_args())
    assert bench.pmc_traffic_bytes(_default_args()) is None


def test_source_hash_covers_the_kernel_and_its_helpers(monkeypatch, tmp_path):
    """Editing either file the attention kernel is built from changes the hash."""
    import os
    import shutil

    csrc = os.path.join(bench.ROOT, "extend-nano-vllm_amd", "csrc")
    fake_root = tmp_path / "repo"
    fake = fake_root / "extend-nano-vllm_amd" / "csrc"
    fake.mkdir(parents=True)
    for name in bench.ATTENTION_SOURCES:
        shutil.copy(os.path.join(csrc, name), fake / name)
    monkeypatch.setattr(bench, "ROOT", str(fake_root))
    h0 = bench.attention_source_hash()
    for name in bench.ATTENTION_SOURCES:
        with open(fake / name, "a") as f:
            f.write("\n// edited\n")
        h1 = bench.attention_source_hash()
        assert h1 != h0
        h0 = h1
