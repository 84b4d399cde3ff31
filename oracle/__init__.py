"""CPU oracle for nano-megatron's vocabulary-parallel cross entropy.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or, for the baseline, as the timed CPU restatement) -- never as the
computation under test. The product path (``nmce``) never imports it and has
no CPU fallback.

Modules
-------
``ce_oracle``   numpy fp64 closed form, per-shard statistics, cross-shard
                combine and gradient (follows nano_megatron/cross_entropy.py),
                and the LM-head projection followed by the loss
                (``lmhead_closed_form``, ``lmhead_sharded``; model.py:192).
``ce_restate``  torch-CPU restatement of the reference's op sequence in fp32,
                used as the timed CPU baseline (``kind: "port"``).

Pinning (what checks each function against something other than itself):
see the module headers; each function lists its checks.
"""
