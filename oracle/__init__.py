"""CPU restatement of Fry's int8 network evaluation -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``chess-transformer_amd/``) imports this package. Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it, and only as the checker (or, for ``cpu_baseline``, as the CPU timing
of the reference algorithm), never as the thing measured or shipped.

Modules:
  int8_ops    -- numpy restatement of the int8 hot-path operators
                 (norm_quant, mix_norm_quant, rotate_quant, int8_linear,
                 template_attention, fp16 linear, Int8Block.forward)
  network     -- the fp32 ChessTransformer forward on the CPU (the
                 reference's CPU path), the input embedding, the heads, and
                 the int8 network forward assembled from int8_ops
"""
