"""CPU oracle for the codebook-dequant MoE expert path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this
package, and only as the checker / the timed CPU restatement.  The product path (the HIP library and the
package's host code) never imports it, and never falls back to it.

Modules (each function cites the reference file:line it restates; paths are relative to
``launcher/glm53-flash/engine/glm53/`` of shallmall/kaggle-llm-endpoint):

* ``bf16``   -- bf16 / f16 bit conversions (round-to-nearest-even), the rounding points of the reference.
* ``iq3s``   -- llama.cpp IQ3_S block dequant (iqquant.py:123-132), the planar packer (planes.py:136-170) and
                the planar dequant (planes.py:262-276), plus the IQ3_S codebook grid.
* ``cb3``    -- the synthetic 3-bit codebook format of the benchmark configs (no reference function exists;
                closed form only).
* ``int8``   -- per-channel int8 weights (quant8.py:26-32) and their bf16 dequant (quant8.py:91-99).
* ``moe``    -- the operator compositions: decode (resident.py:110-120), prefill bookkeeping
                (pallas_moe.py:564-592) and the grouped prefill flow with its bf16 rounding points
                (resident.py:144-165, pallas_moe.py:341-350,622-755), SwiGLU (model.py:119-122).

Pinning: every function is checked in ``tests/test_oracle_*.py`` against the reference's own fixture bytes,
closed-form known-answer cases, an independent second restatement (block form vs planar form), torch as an
independent library for rounding and matmul, and brute force on tiny inputs.
"""
