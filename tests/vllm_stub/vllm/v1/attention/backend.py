"""Stand-ins for vllm.v1.attention.backend (names used by the backend)."""
import enum
from dataclasses import dataclass
from typing import Any, Generic, TypeVar

import torch

M = TypeVar("M")


class AttentionType:
    DECODER = "decoder"
    ENCODER = "encoder"


class AttentionCGSupport(enum.Enum):
    NEVER = 0
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    UNIFORM_BATCH = 2
    ALWAYS = 3


class AttentionBackend:
    pass


class AttentionLayer:
    pass


class AttentionImpl(Generic[M]):
    pass


class AttentionMetadataBuilder(Generic[M]):
    def __init__(self, kv_cache_spec: Any, layer_names: list, vllm_config: Any,
                 device: torch.device) -> None:
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names
        self.vllm_config = vllm_config
        self.device = device
        self.reorder_batch_threshold = None

    def _init_reorder_batch_threshold(self, reorder_batch_threshold: int = 1) -> None:
        self.reorder_batch_threshold = reorder_batch_threshold


@dataclass
class CommonAttentionMetadata:
    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    block_table_tensor: torch.Tensor
    slot_mapping: torch.Tensor
    seq_lens_cpu: torch.Tensor | None = None
