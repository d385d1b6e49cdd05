"""Engine configuration (nanovllm/config.py:14-292, the single-GPU subset).

Kwargs the reference accepts for its other subsystems (data/tensor/pipeline
parallel sizes) are accepted and must be 1: this build runs one GPU, and the
reference itself requires DP=TP=PP=1 for EAGLE3 (config.py:142-149).  Unlike
the reference, an FP8 KV cache may be combined with EAGLE3.  ``load_format``
"dummy" initialises random weights (no checkpoint files needed).
"""
import os
from dataclasses import dataclass

from transformers import AutoConfig


@dataclass
class SpeculativeConfig:
    method: str
    model: str
    num_speculative_tokens: int = 8
    aux_hidden_state_layers: tuple[int, ...] = (2, 18, 33)
    max_model_len: int | None = None

    def __post_init__(self):
        if self.method != "eagle3":
            raise ValueError("only the eagle3 speculative method is supported")
        if not os.path.isdir(self.model):
            raise ValueError(f"speculative model path does not exist: {self.model}")
        if not 1 <= self.num_speculative_tokens <= 8:
            raise ValueError("num_speculative_tokens must be between 1 and 8")
        self.aux_hidden_state_layers = tuple(self.aux_hidden_state_layers)
        if len(self.aux_hidden_state_layers) != 3:
            raise ValueError("EAGLE3 requires exactly three auxiliary hidden layers")


@dataclass
class Config:
    model: str
    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    enable_prefill_batching: bool | None = None
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    data_parallel_size: int = 1
    tensor_parallel_size: int = 1
    pipeline_parallel_size: int = 1
    enforce_eager: bool = False
    enable_prefix_caching: bool = True
    device_offset: int = 0
    hf_config: AutoConfig | None = None
    eos: int = -1
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1
    kv_cache_dtype: str = "auto"
    # physical order inside a KV page: "head_major" stores each kv head's
    # block_size K rows, then its V rows, contiguously ([layers, blocks, Hkv,
    # 2, block_size, D]), which spreads one head's rows over all HBM
    # channels; "token_major" is the reference's [2, layers, blocks,
    # block_size, Hkv, D].  Both are exposed to the layers as the same
    # [blocks, block_size, Hkv, D] K and V views.
    kv_cache_layout: str = "head_major"
    speculative_config: SpeculativeConfig | dict | None = None
    quantization: str | None = None
    load_format: str = "auto"
    seed: int = 0
    # PyTorch TunableOp results (CSV) naming the hipBLASLt / rocBLAS solution
    # for each projection GEMM shape; looked up only, never tuned at run time
    gemm_tuning_file: str | None = None

    def __post_init__(self):
        if not os.path.isdir(self.model):
            raise ValueError(f"model path does not exist: {self.model}")
        if self.kvcache_block_size != 256:
            raise ValueError("kvcache_block_size must be 256")
        if (self.data_parallel_size, self.tensor_parallel_size, self.pipeline_parallel_size) != (1, 1, 1):
            raise ValueError("this build runs on one GPU: data/tensor/pipeline parallel sizes must be 1")
        if self.kv_cache_dtype not in ("auto", "fp8"):
            raise ValueError("kv_cache_dtype must be 'auto' or 'fp8'")
        if self.kv_cache_layout not in ("head_major", "token_major"):
            raise ValueError("kv_cache_layout must be 'head_major' or 'token_major'")
        if self.quantization is not None:
            raise ValueError("weight quantization is not part of this build")
        if self.load_format not in ("auto", "dummy"):
            raise ValueError("load_format must be 'auto' or 'dummy'")
        if self.max_num_batched_tokens <= 0 or self.max_num_seqs <= 0:
            raise ValueError("max_num_batched_tokens and max_num_seqs must be positive")
        if not 0.0 < self.gpu_memory_utilization <= 1.0:
            raise ValueError("gpu_memory_utilization must be in (0, 1]")
        if self.gemm_tuning_file is not None and not os.path.isfile(self.gemm_tuning_file):
            raise ValueError(f"gemm_tuning_file does not exist: {self.gemm_tuning_file}")
        if isinstance(self.speculative_config, dict):
            self.speculative_config = SpeculativeConfig(**self.speculative_config)
        if self.speculative_config is not None:
            if not isinstance(self.speculative_config, SpeculativeConfig):
                raise TypeError("speculative_config must be a SpeculativeConfig or dict")
            self.enable_prefix_caching = False
        self.hf_config = AutoConfig.from_pretrained(self.model)
        if self.hf_config.model_type != "qwen3":
            raise ValueError(f"unsupported model type: {self.hf_config.model_type}")
        if self.enable_prefill_batching is None:
            self.enable_prefill_batching = False
        self.max_model_len = min(self.max_model_len, self.hf_config.max_position_embeddings)
