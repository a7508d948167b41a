"""CPU oracle for the decode-step hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
package. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import, call or link anything here, and only as the
checker or as the timed CPU baseline, never as the thing measured or shipped.

Modules:

* ``int8_quant``      - weight-only int8 format: per-output-channel symmetric
                        absmax quantizer, tile pack/unpack, dequant linear
                        (numpy; bit-exact integer/byte work).
* ``int8_quant.c``    - an independent C restatement of the same quantizer and
                        pack, built by ``oracle/Makefile`` and cross-checked
                        against the numpy one.
* ``paged_attention`` - paged decode attention: SDPA on gathered K/V, the
                        block-loop online softmax, and the fp32 per-row target
                        (torch fp32 on the CPU).
* ``kv_pool``         - the paged KV pool layout and its write/gather
                        (torch on the CPU).
* ``model``           - the fp32 HF decoder (Qwen2 / Llama) holding exactly the
                        device's int8 weights: teacher-forced logits, prefill K/V,
                        continuation from given K/V, greedy decode; used by the
                        greedy-decode and native-step tests.
* ``glue``            - RoPE, RMSNorm + residual, SwiGLU and the KV append of the
                        decode step (torch on the CPU).

Parity status of each function is stated in its module header.
"""
