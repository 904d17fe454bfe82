"""atma_amd -- MI355X (gfx950) implementation of ATMA's global-layer mixer.

The hot path (Polar attention prefill and paged decode, the paged KV write, and
the gated-delta memory's chunked prefill and decode step) runs as hand-written HIP
kernels in ``libatma_hip.so`` behind the C ABI of ``include/atma_hip.h``; the
Python side keeps the reference's op names and signatures:

* ``atma_amd.kernel``  -- polar_attention_fwd, polar_attention_decode,
  gated_delta_decode_step, chunk_gated_delta_rule
* ``atma_amd.layers.attention`` -- store_kvcache, Attention
"""

__version__ = "0.1.0"
