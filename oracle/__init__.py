"""The oracle: a CPU restatement of the reference's speculative-decoding
verify step (Workers-Intelligence-Commons/wpt), in torch on the CPU and FP32.

TEST INFRASTRUCTURE.  Only the tests, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the
checker (or the timed CPU baseline): the product path (wpt_amd) never routes
through it, and fails loudly when its HIP library is missing.

Modules, each citing the reference lines it follows:

    attention  exact (with the top-k choice), sparse (window + chosen rows +
               sink), dense (masked), window attention and the rotary
               encoding: pytorch_kernels.py, attention.py
    cache      the generation cache's rows, readings, KV append, tails and
               undo: cache.py, carry.py
    sampling   the sampling distribution, the acceptance / rejection loop
               (lazily drawn from a torch generator, or read from a tape),
               greedy chain and tree verification, the prefix scheduler:
               wpt_inference/__init__.py
    decoder    the build's generic MQA decoder (random-init weights, exact
               and window layers) behind the reference's model protocol
               new_cache / extend / undo

What pins each function (the checks live in tests/test_oracle_*.py and
tests/test_scheduling.py):

    attention  brute-force formulas one query at a time (the reference's
               exact_by_formula / sparse_by_formula, the choice's sets),
               causality, pieces, padding queries past the table, a
               closed-form single-row case; window attention against the
               pinned sparse form; the rotary encoding by its closed forms
               (identity at position 0, the first and last pairs' angles,
               lengths, relative positions)
    cache      reading in pieces equals reading whole; undo of the reference's
               kept patterns equals reading only the kept tokens (exact and
               window layers)
    sampling   multinomial = argmax(w / Exp(1)) with the generator state;
               greedy = top_k 1; a recorded lazy run replayed through the
               tape gives the same decisions; statistical: uniform drafts keep
               the model's distribution (total variation < 0.05 over 4000
               rows); the scheduler's known answers (test_sampling.py:230-238)
               and a brute force over widths
The exact token stream the reference's Writer draws from a seed through its
lazy generator order (its own tests assert only "same seed, same tokens") is
pinned by golden streams of the reference's Writer itself
(tests/golden/writer_vectors.json, written by
tests/golden/make_writer_vectors.py on the stub model of tests/golden/stubs.py):
the oracle's lazy replay writes the same tokens and counts
(tests/test_oracle_writer.py).
"""
