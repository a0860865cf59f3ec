"""Oracle of the draws a torch generator on the GPU makes (test
infrastructure; see oracle/__init__.py): the stream the reference's Writer
consumes when its generator lives on the GPU, restated on the CPU with numpy.

The reference draws from torch, a dependency absent from the reference tree
(torch 2.10 with ROCm here); its call sites are
packages/wpt-inference/src/wpt_inference/__init__.py:214 (torch.rand(()) per
draft judged), :219 and :222 (torch.multinomial(w, 1)) and :181-182
(Writer._sample: one torch.multinomial over every row).  What those draw:

    philox4x32_10   the block generator (Salmon, Moraes, Dror and Shaw,
                    "Parallel random numbers: as easy as 1, 2, 3", SC 2011):
                    a 128-bit counter (its low half the block index, its high
                    half the subsequence) under the 64-bit seed
    threads         a draw of numel floats runs S = 256 min(CUs x (max
                    threads a CU / 256), ceil(numel / 256)) threads
    uniforms        thread t takes block offset / 4 + k of subsequence t and
                    gives entry 4 S k + S w + t its word w, as (word + 1)
                    2^-32 rounded to float (in (0, 1]); the call moves the
                    offset on by step(numel) = 4 ceil(numel / 4 S)
    rand_scalar     torch.rand(()): entry 0 of a draw of one, 1 read as 0
    exponentials    Exp(1) as torch forms them on the device, -log u (u at or
                    above 1 - 2^-24 giving 2^-24); here with numpy's log, which
                    may differ from the device's logf in the last bits (the GPU
                    test compares the kernel with torch itself)

Pinned by tests/test_oracle_philox.py against values torch's generator drew
on an MI355X (tests/golden/torch_gpu_draws.json, written by
tests/golden/make_torch_gpu_draws.py).
"""

import numpy as np

_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)


def philox4x32_10(block, subsequence, seed):
    """The four 32-bit words (..., 4) of counter (block, subsequence) under
    seed; block and subsequence are arrays of 64-bit values."""
    block = np.asarray(block, dtype=np.uint64)
    subsequence = np.asarray(subsequence, dtype=np.uint64)
    block, subsequence = np.broadcast_arrays(block, subsequence)
    c0 = (block & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    c1 = (block >> np.uint64(32)).astype(np.uint32)
    c2 = (subsequence & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    c3 = (subsequence >> np.uint64(32)).astype(np.uint32)
    k0, k1 = np.uint32(seed & 0xFFFFFFFF), np.uint32(seed >> 32)
    with np.errstate(over="ignore"):
        for _ in range(10):
            p0 = _M0 * c0.astype(np.uint64)
            p1 = _M1 * c2.astype(np.uint64)
            c0, c1, c2, c3 = ((p1 >> np.uint64(32)).astype(np.uint32) ^ c1 ^ k0, p1.astype(np.uint32),
                              (p0 >> np.uint64(32)).astype(np.uint32) ^ c3 ^ k1, p0.astype(np.uint32))
            k0, k1 = k0 + _W0, k1 + _W1
    return np.stack([c0, c1, c2, c3], -1)


def threads(numel, cus=256, threads_per_cu=2048):
    """S: the threads torch runs for a draw of numel floats."""
    return 256 * min(cus * (threads_per_cu // 256), (numel + 255) // 256)


def step(numel, cus=256, threads_per_cu=2048):
    """How far a draw of numel floats moves the generator's offset."""
    return 4 * ((numel - 1) // (4 * threads(numel, cus, threads_per_cu)) + 1)


def uniforms(seed, offset, numel, cus=256, threads_per_cu=2048):
    """The float32 uniforms in (0, 1] of a draw of numel entries at offset."""
    S = threads(numel, cus, threads_per_cu)
    li = np.arange(numel, dtype=np.int64)
    k, rest = li // (4 * S), li % (4 * S)
    word, t = rest // S, rest % S
    words = philox4x32_10(offset // 4 + k, t, seed)[np.arange(numel), word]
    return np.float32(2.0 ** -32) + words.astype(np.float32) * np.float32(2.0 ** -32)


def rand_scalar(seed, offset):
    """torch.rand(()) at offset."""
    u = uniforms(seed, offset, 1)[0]
    return np.float32(0.0) if u == 1 else u


def exponentials(seed, offset, numel, cus=256, threads_per_cu=2048):
    """Exp(1) of a draw of numel entries at offset (float32; numpy's log)."""
    u = uniforms(seed, offset, numel, cus, threads_per_cu)
    edge = np.float32(2.0 ** -24)
    log = np.where(u >= np.float32(1) - edge, -edge, np.log(u.astype(np.float64)).astype(np.float32))
    return (-log).astype(np.float32)
