"""CPU oracle for the Mira mixer scan -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
anything from this package, and only as the checker (or, in bench.py, as the timed CPU
baseline). The product path (`official-mira-llm_amd/mira_amd`) never imports it and fails
loudly when its HIP library is missing.

Modules:
  lattice   -- restatement of the reference operator `matrix_lattice_iir` (stage maps, the
               sequential stage loop, the batched per-token formulation, the per-token affine
               system and the chunked (Phi, S) emulation).
  baseline  -- the BASELINE-literal closed forms (depthwise causal conv + diagonal scan with a
               ring buffer, GLA matrix state) and their exact K=1 realisations as lattice inputs.

Every function names the reference file:line it restates. Pinning (what checks each function
against something other than itself) lives in tests/test_oracle.py; functions with no such
check say "parity unpinned" in their docstring.
"""
