"""CPU oracle for flash-eq's equivariant edge hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (``flash-eq_amd/``)
may import, link or execute anything under ``oracle/``; only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and
only as the checker / CPU baseline, never as the thing measured or shipped.

Contents (each function cites the reference ``file:line`` it restates):

* ``layout``     -- irrep metadata, m-first permutation, block parameters.
* ``wigner``     -- so(3) generators, ``WignerD.rot``/``rot_to_ez``,
                    ``WignerDBasis`` via ``torch.linalg.matrix_exp`` in float64.
* ``blockdiag``  -- the block-diagonal radial mix, forward and backward, in two
                    independent forms: dense per-edge Lambda (float64, tiny E)
                    and bin-grouped BLAS (any dtype, large E; the CPU baseline).
* ``cref``       -- ctypes wrapper of ``blockdiag_ref.c``, a third form that
                    follows the CUDA kernels' per-edge loops and float32 binning.
* ``radial``     -- ``SeparableRadialNet`` table formula.
* ``graphops``   -- sum pooling and the per-destination edge softmax.
* ``layer``      -- ``EquivariantEdgewiseLinear`` / attention composition.

Pinning status of every function is recorded in its docstring ("pinned by"
lists the tests under ``tests/`` that check it against golden vectors,
known-answer tests, closed forms or invariants).
"""
