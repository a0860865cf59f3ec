"""The oracle: a CPU restatement of the reference's speculative-decoding
verify step (Workers-Intelligence-Commons/wpt), in torch on the CPU and FP32.

TEST INFRASTRUCTURE.  Only the tests, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the
checker (or the timed CPU baseline): the product path (wpt_amd) never routes
through it, and fails loudly when its HIP library is missing.

Modules, each citing the reference lines it follows:

    attention  exact, sparse (window + chosen rows + sink) and dense (masked)
               attention: pytorch_kernels.py, attention.py
    cache      the generation cache's rows, readings, KV append and undo:
               cache.py, carry.py
    sampling   the sampling distribution, the acceptance / rejection loop
               (lazily drawn from a torch generator, or read from a tape),
               greedy chain and tree verification: wpt_inference/__init__.py
    decoder    the build's generic MQA decoder (random-init weights) behind
               the reference's model protocol new_cache / extend / undo
    writer     the reference's Writer (speculative writing) over that protocol

What pins each function (the checks live in tests/test_oracle_*.py):

    attention  brute-force formulas one query at a time (the reference's
               exact_by_formula / sparse_by_formula), causality, pieces,
               padding queries past the table, a closed-form single-row case
    cache      reading in pieces equals reading whole; undo of the reference's
               kept patterns equals reading only the kept tokens
    sampling   the reference's schedule known answers; greedy = top_k 1;
               multinomial = argmax(w / Exp(1)) with the generator state;
               a recorded lazy run replayed through the tape gives the same
               decisions; statistical: uniform drafts keep the model's
               distribution (total variation < 0.05 over 4000 rows)
    writer     golden vectors from the reference's own Writer
               (tests/golden/writer_vectors.json, made by
               tests/golden/make_writer_vectors.py)
"""
