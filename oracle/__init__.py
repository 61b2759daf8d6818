"""CPU oracle for the population-perturbed forward: TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU, the reference's algorithm for the hot path
(`train/val/eggroll.py:38-168` and the helpers of `utils/model.py:14-210`). It exists to check the
MI355X HIP path and nothing else:

* only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it;
* the product package `noise_amd` never imports it and never falls back to it.

Modules:
  model    -- norm, rotary, windowed attention, lowrank / lowrank_embed, population_loss,
              clean forward (the P=1, sigma=0 case), credit moments.
  eggroll  -- noise buffer offsets, fitness, update reconstruction, Adam step.

Every function cites the reference file:line it follows. Parity pins (how each function is itself
checked) are listed in the module docstrings; a function without one says "parity unpinned".
"""
