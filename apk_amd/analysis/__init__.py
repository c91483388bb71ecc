"""Post-processing of the binaries' latency CSVs and OBS1 matrices.

CPU-only analyses over what `yield --mode latency|visibility --csv
--dump-obs` writes, restated from the reference's scripts for this build's
files (nearest-rank percentiles, warm-up events discarded), plus the engine
clock read-back under load:

- spread:         observation spread per event and the identity
                  lat == first-observer delay + spread
                  (reference scripts/reanalyze_spread.py)
- maxofn:         held-out max-of-N independence model and the every-event
                  floor check (reference scripts/heldout_maxofn.py)
- visibility:     Dmax p50/p99 per visibility matrix
                  (reference scripts/make_visibility_summary.py)
- clock_readback: the engine clock sampled with rocm-smi while a GEMM load
                  runs (reference scripts/lock_clocks.sh:15-25)

Nothing here loads the HIP library.
"""
