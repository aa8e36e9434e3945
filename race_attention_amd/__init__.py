"""race_attention_amd -- MI355X (gfx950) RACE attention operator.

Hand-written HIP kernels behind a C ABI (include/race_attention.h), with
PyTorch modules mirroring the reference API:
  race_attention_amd.race  causal BatchedACE / RACEAttention / RACEBlock /
                           RACEPrefixMeanFlatFn   (misc/race.py)
  race_attention_amd.vit   non-causal BatchedACE / RACEAttention / RACEBlock
                           (misc/vit.py)
  race_attention_amd.causal  globally normalised CausalRACEAttention
                           (misc/elsaa_causal_complete.py)
  race_attention_amd.functional  race_attention(), race_attention_global(),
                           RACEFunction, RACEGlobalFunction, raw calls
"""
from .functional import (RACEFunction, RACEGlobalFunction, RACEPrefixMeanFlatFn, race_attention,  # noqa: F401
                         race_attention_global)

__all__ = ["RACEFunction", "RACEGlobalFunction", "RACEPrefixMeanFlatFn", "race_attention", "race_attention_global"]
