"""CPU oracle for SignRot's W4A4 real-quant path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's real-quant
path (HYU-ARK-Lab/SignRot, `signrot/` + `fake_quant/`), each function citing
the reference file:line it follows.  It exists to check the HIP kernels and
nothing else: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only as the checker (or,
for `cpu_baseline`, as the timed CPU restatement).  The shipped package
`signrot_amd` never imports it; with the HIP library missing the product
path raises instead of falling back here.

Pinning (how each function is checked independently of its own formula;
the checks live in tests/test_oracle_*.py):

* hadamard.get_hadK / tables   -- Hadamard property H Hᵀ = K·I, ±1 entries,
                                   SHA-256 of the tables parsed from the
                                   reference text, known answers for the
                                   config widths.
* hadamard.fwht                -- scipy.linalg.hadamard brute force (float64).
* hadamard.rotate              -- Kronecker closed form np.kron(H_K, H_{n/K})
                                   within the two fp16 rounding points.
* quant.sym_quant_dynamic      -- exact rational arithmetic (fractions) for
                                   the fp16 quotient and round-half-even, the
                                   reference's edge cases (zeros, spike, range,
                                   tiny, all-negative), code-range invariants.
* quant.pack_i4 / unpack_i4    -- hand-computed bytes, round-trip identity.
* quant.matmul_s4s4            -- brute-force Python-int triple loop.
* quant.sym_dequant            -- Python double arithmetic with explicit
                                   fp32 rounding through struct.
* quant.kv_quant_pack          -- constant-row case, reconstruction bound
                                   |x - x̂| <= scale/2 (+ fp16 slack).
* attention.decode             -- float64 softmax attention, split vs unsplit.
* glue.*                       -- float64 restatements within ulp bounds.

Functions whose exact bits no available artefact fixes (the reference's
fast_hadamard_transform FWHT order and cuBLAS's fp16 `hadK @ x`) are pinned by
tolerance only: "parity unpinned" at the bit level for the rotation, which is
why integer parity is defined on the rotated fp16 input.
"""
