"""Model folders: the decoder's weights saved and loaded in the reference's
layout (packages/wpt-model/src/wpt_model/checkpoint.py:1-204), the Hugging
Face one:

    config.json                          the decoder's numbers (DecoderConfig)
    model.safetensors                    every weight, when not split
    model-00001-of-00003.safetensors     or one file per shard,
    model.safetensors.index.json         plus the index: tensor name -> file
    tokenizer.json                       the vocabulary the weights were trained with
    drafter/                             the drafter trained against these weights

Every weight file's header names the tokenizer (`tokenizer`) and the sha256
of tokenizer.json (`tokenizer_sha256`); load_tokenizer refuses a
tokenizer.json that does not match (TokenizerMismatch, :146-158).  A model
and its drafter are one unit: load_decoder refuses a folder whose drafter is
missing, was not saved whole, or names other weights by their sha256
(DrafterMismatch, :110-125).  safetensors holds only tensors, so loading runs
nothing from the files.

The weights are the decoder's (wpt_amd.decoder.random_weights' names); this
build has no drafter model, so a folder's drafter/ is checked, not loaded
(save_drafter_record writes the part the check reads: its config.json and
provenance.json).
"""

import dataclasses
import hashlib
import json
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import load_file, save_file

from .decoder import DecoderConfig, MQADecoder

CONFIG_NAME = "config.json"
SINGLE_NAME = "model.safetensors"
INDEX_NAME = "model.safetensors.index.json"
TOKENIZER_NAME = "tokenizer.json"
DRAFTER_NAME = "drafter"
METADATA = {"format": "pt"}
CHUNK = 1 << 20


class DrafterMismatch(ValueError):
    """The model folder has no drafter, or its drafter was trained against
    other weights than the folder's."""


class TokenizerMismatch(ValueError):
    """tokenizer.json is missing or is not the vocabulary the weight files'
    headers name (or the headers name none, or disagree)."""


def sha256_file(path):
    """The sha256 of a file, 64 lowercase hex digits (read in 1 MiB blocks)."""
    digest = hashlib.sha256()
    with open(path, "rb") as f:
        while block := f.read(CHUNK):
            digest.update(block)
    return digest.hexdigest()


def save_folder(config, weights, directory, tokenizer, tokenizer_name, max_shard_bytes=None, metadata=None):
    """Writes the model folder, replacing any model saved there: the weights
    (a dict of tensors) in one file, or packed in order into files of at most
    max_shard_bytes (a larger tensor gets a file of its own) with the index;
    tokenizer.json (the bytes `tokenizer`, named tokenizer_name in every
    file's header); config.json last, so that a save that stops midway
    leaves a folder load_decoder refuses."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    _remove(directory)
    state = {name: value.detach().cpu().contiguous() for name, value in weights.items()}
    header = {**(metadata or {}), "tokenizer": tokenizer_name,
              "tokenizer_sha256": hashlib.sha256(tokenizer).hexdigest(), **METADATA}
    (directory / TOKENIZER_NAME).write_bytes(tokenizer)
    shards = _split(state, max_shard_bytes)
    if len(shards) == 1:
        save_file(shards[0], directory / SINGLE_NAME, metadata=header)
    else:
        weight_map = {}
        for i, shard in enumerate(shards, start=1):
            name = f"model-{i:05d}-of-{len(shards):05d}.safetensors"
            save_file(shard, directory / name, metadata=header)
            weight_map.update({key: name for key in shard})
        index = {"metadata": {"total_size": sum(_nbytes(t) for t in state.values())}, "weight_map": weight_map}
        (directory / INDEX_NAME).write_text(json.dumps(index, indent=2) + "\n", encoding="utf-8", newline="\n")
    (directory / CONFIG_NAME).write_text(json.dumps(dataclasses.asdict(config), indent=2) + "\n", encoding="utf-8",
                                         newline="\n")


def load_config(directory):
    """The DecoderConfig of config.json."""
    fields = json.loads((Path(directory) / CONFIG_NAME).read_text(encoding="utf-8"))
    fields["kinds"] = tuple(fields.get("kinds", ()))
    return DecoderConfig(**fields)


def load_weights(directory):
    """(config, weights on the CPU) of a model folder; DrafterMismatch when
    its drafter is missing or was trained against other weights."""
    directory = Path(directory)
    check_drafter(directory)
    config = load_config(directory)
    weights = {}
    for name in weight_files(directory):
        weights.update(load_file(directory / name))
    return config, weights


def load_decoder(directory, dtype=torch.bfloat16, device="cuda"):
    """The decoder of a model folder, on the GPU (the reference's load_model,
    checkpoint.py:97-107)."""
    config, weights = load_weights(directory)
    return MQADecoder(config, weights, dtype=dtype, device=device)


def check_drafter(directory):
    """DrafterMismatch unless the folder holds a drafter whose provenance
    names the folder's weights, by their sha256, as those it was trained
    against (checkpoint.py:110-125)."""
    directory = Path(directory)
    drafter = directory / DRAFTER_NAME
    try:
        provenance = json.loads((drafter / "provenance.json").read_text(encoding="utf-8"))
    except FileNotFoundError:
        raise DrafterMismatch(f"{directory}: no drafter ({DRAFTER_NAME}/); a model folder holds the drafter "
                              "trained for its weights") from None
    if not (drafter / CONFIG_NAME).exists():
        raise DrafterMismatch(f"{directory}: its drafter ({DRAFTER_NAME}/) was not saved whole")
    trained = (provenance.get("target") or {}).get("weights")
    weights = weight_hashes(directory)
    if trained != weights:
        raise DrafterMismatch(f"{directory}: its drafter was trained against weights {trained}, the folder holds "
                              f"{weights}; train the model again to train its drafter")


def save_drafter_record(directory, config=None, provenance=None):
    """drafter/config.json and drafter/provenance.json, naming the folder's
    current weights as those the drafter was trained against unless
    provenance is given."""
    drafter = Path(directory) / DRAFTER_NAME
    drafter.mkdir(parents=True, exist_ok=True)
    if provenance is None:
        provenance = {"target": {"weights": weight_hashes(directory)}}
    (drafter / "provenance.json").write_text(json.dumps(provenance, indent=2) + "\n", encoding="utf-8")
    (drafter / CONFIG_NAME).write_text(json.dumps(config or {}, indent=2) + "\n", encoding="utf-8")


def tokenizer_identity(directory):
    """(tokenizer name, sha256 of tokenizer.json) as the weight files'
    headers name them (checkpoint.py:128-143)."""
    directory = Path(directory)
    found = set()
    for name in weight_files(directory):
        with safe_open(directory / name, framework="pt") as weights:
            header = weights.metadata() or {}
        found.add((header.get("tokenizer"), header.get("tokenizer_sha256")))
    if len(found) != 1 or None in next(iter(found)):
        raise TokenizerMismatch(f"{directory}: the weight files name no single tokenizer ({sorted(found, key=str)})")
    return next(iter(found))


def load_tokenizer(directory):
    """The bytes of tokenizer.json, only when they are the vocabulary the
    weights name (checkpoint.py:146-158)."""
    directory = Path(directory)
    name, expected = tokenizer_identity(directory)
    try:
        data = (directory / TOKENIZER_NAME).read_bytes()
    except FileNotFoundError:
        raise TokenizerMismatch(f"{directory}: no {TOKENIZER_NAME}; the weights need tokenizer {name}") from None
    actual = hashlib.sha256(data).hexdigest()
    if actual != expected:
        raise TokenizerMismatch(f"{directory}: {TOKENIZER_NAME} has sha256 {actual}, but the weights were trained "
                                f"with tokenizer {name}, sha256 {expected}")
    return data


def weight_files(directory):
    """The folder's weight files, sorted: model.safetensors, or the shards
    its index names (checkpoint.py:161-169)."""
    index = Path(directory) / INDEX_NAME
    if index.exists():
        return sorted(set(json.loads(index.read_text(encoding="utf-8"))["weight_map"].values()))
    return [SINGLE_NAME]


def weight_hashes(directory):
    """{file name: sha256} of each weight file."""
    directory = Path(directory)
    return {name: sha256_file(directory / name) for name in weight_files(directory)}


def _split(state, max_shard_bytes):
    if max_shard_bytes is None:
        return [state]
    shards, current, size = [], {}, 0
    for key, tensor in state.items():
        n = _nbytes(tensor)
        if current and size + n > max_shard_bytes:
            shards.append(current)
            current, size = {}, 0
        current[key] = tensor
        size += n
    shards.append(current)
    return shards


def _nbytes(tensor):
    return tensor.numel() * tensor.element_size()


def _remove(directory):
    for path in directory.glob("model*.safetensors"):
        path.unlink()
    for name in (INDEX_NAME, CONFIG_NAME, TOKENIZER_NAME):
        (directory / name).unlink(missing_ok=True)
