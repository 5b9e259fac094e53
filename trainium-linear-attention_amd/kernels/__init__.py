"""MI355X (gfx950) BASED linear attention: host-side mirror of the reference's kernel
wrappers, backed by libbased_la.so (HIP kernels behind a C ABI)."""

from .based_layer import based_layer_attn
from .based_module import TrainiumBasedLinearAttention, TrainiumBasedLinearAttentionNKI
from .chunked_attention import (based_chunked, based_decode_step, chunked_based_attn, chunked_nki_numerator,
                                feature_dim, taylor_feature_map)
from .identity_attention import identity_linear_attn
from .pytorch_attention import based_parallel, solution, solution_nki
from .sliding_attention import nki_sliding_window_attn, sliding_window_attn

__all__ = [
    "solution_nki", "solution", "based_parallel",
    "taylor_feature_map", "feature_dim", "chunked_nki_numerator", "chunked_based_attn", "based_chunked",
    "nki_sliding_window_attn", "sliding_window_attn",
    "TrainiumBasedLinearAttention", "TrainiumBasedLinearAttentionNKI", "based_layer_attn",
    "identity_linear_attn", "based_decode_step",
]
