"""CPU oracle for the iPC training step (test infrastructure only).

This package restates the reference's pure-PyTorch fp32 algorithm
(``src/ipc_tilelang/reference.py``, ``src/ipc_tilelang/activations.py``,
``src/ipc_tilelang/trainer.py:453-516``) so that the HIP path can be checked
against it on identical seeded inputs.

It is a checker, never a product path: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
import it.  ``lich_amd`` never imports anything from here and has no CPU
fallback.

Modules
-------
``ipc_oracle``  torch fp32 (or fp64) restatement of the reference step.
``ipc_brute``   independent pure-Python float64 loops over the README
                equations, used to pin ``ipc_oracle`` on tiny shapes.
``emulate``     storage/operand precision emulator (rounds at the points the
                HIP kernels round) used to fix the 16-bit tolerances.
"""
