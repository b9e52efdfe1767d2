"""CPU oracle for the resident decode epoch.

TEST INFRASTRUCTURE ONLY.  Nothing under ``oracle/`` is part of the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and there only as the checker (or, for the CPU
baseline, as the thing timed on the host cores).  The HIP library never calls
into it and the product path raises when the HIP library is missing.

Modules (each function cites the reference file:line it restates):

* ``decoder``    -- ``PagedQwenDecoderStep`` (history/attempts/
  g4c-attempt69b-b4-eager/batched_decoder_step.py:197-417), parametric in the
  model dims, dtype and paged-KV geometry.
* ``controller`` -- ``G4cB4ResidentEpoch::Proc`` (controller/
  g4c_b4_resident_epoch.cpp:84-622), the K-step epoch with its validation,
  resident state, argmax and EOS logic.
* ``bridge``     -- ``resident_epoch_execute`` packing/unpacking
  (native/resident_epoch_bridge.cpp:350-357, 424-649).
* ``weights``    -- seeded N(0, 0.02) weights in the reference bundle naming
  (materialize_runtime_weights.py:53-80).
* ``workloads``  -- the five workload configurations.
* ``hf_reference`` -- the reference's own acceptance oracle, HF
  ``Qwen2ForCausalLM`` eager (batched_decoder_step.py:477-518), built from a
  local config with the same weights.

Parity pinning status is recorded per function in each module docstring.
"""
