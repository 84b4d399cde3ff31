"""nmce: nano-megatron's vocabulary-parallel cross entropy on MI355X (gfx950).

Public API (mirrors nano_megatron/cross_entropy.py and parallel.py):

* ``vocab_parallel_cross_entropy(logits, target, vocab_start, vocab_end, ctx)``
  -> mean fp32 loss; backward yields the logits gradient.
* ``_VocabParallelCrossEntropy`` -- the autograd Function (per-token loss).
* ``lmhead_vocab_parallel_cross_entropy(hidden, weight, target, vocab_start,
  vocab_end, ctx)`` -> the same loss of ``hidden @ weight.t()`` (the LM head of
  model.py:192 fused in), never storing the logits; backward yields the hidden
  and weight gradients.
* ``FusedParallelLMHead(config, ctx)`` -- drop-in for model.py's
  ``ParallelLMHead`` whose ``forward(x, labels)`` returns that fused loss.
* ``copy_to_tensor_parallel_region`` / ``gather_from_sequence_parallel_region``
  / ``gather_tokens_rank_major`` -- the collectives on the LM head's input side
  (mappings.py:83-94, :109-120).
* ``ParallelContext`` / ``vocab_range`` / ``divide`` -- the topology fields and
  shard rule the loss reads.

All loss compute runs in ``libnmce.so`` (hand-written HIP for gfx950) through the C
ABI in ``include/nmce.h``; there is no CPU or PyTorch fallback.
"""

from .cross_entropy import (
    _VocabParallelCrossEntropy,
    validate_targets,
    vocab_parallel_cross_entropy,
)
from .lmhead import (
    FusedParallelLMHead,
    _LMHeadVocabParallelCrossEntropy,
    lmhead_vocab_parallel_cross_entropy,
)
from .mappings import (
    copy_to_tensor_parallel_region,
    gather_from_sequence_parallel_region,
    gather_tokens_rank_major,
    targets_rank_major,
)
from .parallel import ParallelContext, divide, vocab_range

__all__ = [
    "FusedParallelLMHead",
    "_LMHeadVocabParallelCrossEntropy",
    "_VocabParallelCrossEntropy",
    "ParallelContext",
    "copy_to_tensor_parallel_region",
    "divide",
    "gather_from_sequence_parallel_region",
    "gather_tokens_rank_major",
    "lmhead_vocab_parallel_cross_entropy",
    "targets_rank_major",
    "validate_targets",
    "vocab_parallel_cross_entropy",
    "vocab_range",
]
