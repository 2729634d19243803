"""gfx950 HIP kernels of the index-resident multi-adapter LoRA path (API of ``lithe.kernels``).

* ``packed``  9-bit index packing (7 indices per uint64 word), unpacking and the
              bulk decode from the packed GPU-resident form.
* ``shared``  index-resident per-sample LoRA delta: the decode is fused into the
              shrink / expand tiles, reading one codebook shared by all samples.
* ``sgmv``    per-sample LoRA delta over decoded (dense) factors.
* ``layers``  ``nn.Module`` wrappers that route each sample of a batch to its own
              adapter with the kernels above.
* ``bank``    a contiguous GPU-resident bank of packed adapters.

Everything here runs on the GPU through ``liblithe_amd.so``; there is no CPU
fallback. ``HAS_HIP`` says whether the library is built and loadable. The
reference's ``*_reference`` PyTorch functions are not part of this package:
their restatement is the test oracle under ``oracle/``.
"""
from ._hip import HAS_HIP, gpu_available, workspace_errors
from .bank import PackedBank
from .layers import IndexLoRALinear, PerSampleLoRALinear, wrap_linears
from .packed import (PackedLayout, blockify_factors, decode_int16, decode_packed, decode_packed_slots, decode_packed_stacked,
                     flat_indices, pack_adapter, pack_indices, split_decoded, split_stacked, unpack_indices)
from .sgmv import per_sample_lora_delta
from .shared import packed_lora_delta, shared_codebook_lora_delta

__all__ = [
    "HAS_HIP", "gpu_available", "workspace_errors",
    "IndexLoRALinear", "PerSampleLoRALinear", "wrap_linears", "PackedBank",
    "PackedLayout", "blockify_factors", "decode_packed", "decode_packed_slots", "decode_packed_stacked", "decode_int16",
    "flat_indices", "pack_adapter", "pack_indices", "split_decoded", "split_stacked", "unpack_indices",
    "per_sample_lora_delta", "packed_lora_delta", "shared_codebook_lora_delta",
]
