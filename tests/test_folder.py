"""Model folders on the CPU, as the reference's own checkpoint tests read them
(packages/wpt-model/tests/test_checkpoint.py:18-72): a split folder loads
back identical, a folder loads only with the drafter trained against its
weights, and only with the vocabulary its weights name."""

import hashlib
import json

import pytest
import torch

from wpt_amd import folder
from wpt_amd.decoder import DecoderConfig, layer_kinds, random_weights

VOCABULARY = b'{"format":"wpt-bpe","merges":[],"tokenizer_version":"0.2.0"}\n'
KINDS = layer_kinds(1, 1, 1)
TINY = DecoderConfig(layers=len(KINDS), d_model=64, heads=2, head_dim=64, ffn=96, vocab=50, kinds=KINDS, window=16,
                     rope_dims=32, top_k=8)


def test_a_split_folder_loads_back_identical(tmp_path):
    weights = random_weights(TINY, dtype=torch.bfloat16)
    folder.save_folder(TINY, weights, tmp_path, VOCABULARY, "test version 1", max_shard_bytes=20_000)
    folder.save_drafter_record(tmp_path)
    assert len(list(tmp_path.glob("model-*-of-*.safetensors"))) > 1
    index = json.loads((tmp_path / folder.INDEX_NAME).read_text())
    assert set(index["weight_map"]) == set(weights)
    config, loaded = folder.load_weights(tmp_path)
    assert config == TINY and loaded.keys() == weights.keys()
    assert all(torch.equal(weights[k], loaded[k]) and weights[k].dtype == loaded[k].dtype for k in weights)
    # the tokenizer is named in every shard
    assert folder.tokenizer_identity(tmp_path) == ("test version 1", hashlib.sha256(VOCABULARY).hexdigest())


def test_one_file_when_not_split(tmp_path):
    weights = random_weights(TINY)
    folder.save_folder(TINY, weights, tmp_path, VOCABULARY, "test version 1")
    assert folder.weight_files(tmp_path) == [folder.SINGLE_NAME] and not (tmp_path / folder.INDEX_NAME).exists()
    folder.save_drafter_record(tmp_path)
    _, loaded = folder.load_weights(tmp_path)
    assert all(torch.equal(weights[k], loaded[k]) for k in weights)


def test_a_folder_loads_only_with_the_drafter_trained_against_its_weights(tmp_path):
    weights = random_weights(TINY)
    folder.save_folder(TINY, weights, tmp_path, VOCABULARY, "test version 1")
    with pytest.raises(folder.DrafterMismatch, match="no drafter"):
        folder.load_weights(tmp_path)
    folder.save_drafter_record(tmp_path)
    folder.load_weights(tmp_path)
    weights["layers.0.attn_norm"] = weights["layers.0.attn_norm"] + 0.5  # other weights in the same folder
    folder.save_folder(TINY, weights, tmp_path, VOCABULARY, "test version 1")
    with pytest.raises(folder.DrafterMismatch, match="trained against weights"):
        folder.load_weights(tmp_path)
    folder.save_drafter_record(tmp_path)
    (tmp_path / "drafter" / "config.json").unlink()  # a save that stopped midway
    with pytest.raises(folder.DrafterMismatch, match="not saved whole"):
        folder.load_weights(tmp_path)


def test_a_folder_runs_only_with_the_vocabulary_its_weights_name(tmp_path):
    folder.save_folder(TINY, random_weights(TINY), tmp_path, VOCABULARY, "test version 1")
    assert folder.load_tokenizer(tmp_path) == VOCABULARY
    (tmp_path / "tokenizer.json").write_bytes(VOCABULARY.replace(b"0.2.0", b"0.3.0"))
    with pytest.raises(folder.TokenizerMismatch, match="trained with tokenizer test version 1"):
        folder.load_tokenizer(tmp_path)
    (tmp_path / "tokenizer.json").unlink()
    with pytest.raises(folder.TokenizerMismatch, match="no tokenizer.json"):
        folder.load_tokenizer(tmp_path)


def test_the_file_hashes_are_the_files_sha256(tmp_path):
    folder.save_folder(TINY, random_weights(TINY), tmp_path, VOCABULARY, "v", max_shard_bytes=50_000)
    hashes = folder.weight_hashes(tmp_path)
    assert hashes == {name: hashlib.sha256((tmp_path / name).read_bytes()).hexdigest() for name in hashes}
