"""CPU oracle for the index-resident multi-adapter LoRA path.

TEST INFRASTRUCTURE ONLY. This package is a plain numpy (plus one small C
file) restatement of the reference algorithm, written from the reference's
source and README specification. It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
there only as the checker. The product (``lithe_amd``) never imports it and has
no CPU fallback: its entry points raise when the HIP library or a GPU tensor is
missing.

Modules (each function cites the reference file:line it restates; paths are
relative to the reference repository root):

* ``codebook``  the Sylvester-Hadamard 9-bit twin codebook and pools
                (``lithe/codebook.py``).
* ``packing``   9-bit x 7-per-word packing, ``PackedLayout`` offsets and the
                packed-stream order (``lithe/kernels/packed.py``).
* ``decode``    L-level residual decode in fp32 (level order) and the fp32 ->
                bf16 round-to-nearest-even cast (``lithe/quant.py``,
                ``lithe/kernels/packed.py``).
* ``delta``     the per-sample LoRA deltas with the reference's dtype steps:
                ``shared_codebook_lora_delta_reference``, the serve.py
                rank-stacked routing, ``per_sample_lora_delta`` and
                ``LitheLinear`` inference.
* ``native``    ctypes binding of ``oracle/c/lithe_oracle.c``, an independent C
                restatement of pack / unpack / decode used to cross-check the
                numpy restatement bit for bit and as the CPU baseline.

How each function is pinned (no reference import is needed; every function is
closed form):

* codebook: the SHA-256 of the integer table from the reference tests,
  ``scipy.linalg.hadamard`` (a library Sylvester construction), orthogonality.
* packing: the Kohya-304 size known-answer test (3,589,632 indices ->
  4,102,440 bytes), hand-computed words, round trips, the C restatement.
* decode: brute force from the Hadamard matrix in float64, the all-equal-index
  special case, the C restatement, torch's own bf16 cast.
* delta: float64 closed forms (decode-then-matmul, per-route sums with the
  mixture weights) and planted-mistake checks.
"""
