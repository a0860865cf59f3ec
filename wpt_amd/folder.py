"""Model folders for the decoder.

On-disk format (kept identical to the reference's model folders,
packages/wpt-model/src/wpt_model/checkpoint.py:1-21, so that a folder written
by either names its weights, vocabulary and drafter the same way):

    config.json                          DecoderConfig's fields
    model.safetensors                    the weights, in one file
    model-00001-of-00003.safetensors     or in numbered parts,
    model.safetensors.index.json         {"metadata": {"total_size": bytes},
                                          "weight_map": {tensor: file}}
    tokenizer.json                       the vocabulary's bytes
    drafter/config.json                  the drafter's numbers
    drafter/provenance.json              {"target": {"weights": {file: sha256}}}

Each weight file's safetensors header carries `tokenizer` (the vocabulary's
name), `tokenizer_sha256` (the sha256 of tokenizer.json) and `format: pt`.
Parts are filled in the weights' own order and a new part starts when the
next tensor would push the current one past the limit (a tensor larger than
the limit sits alone).

Design: a `ModelFolder` object owns one directory.  Writing puts the weight
shards and tokenizer.json in place first and config.json last (the JSON files
each written under a temporary name and renamed into place), so a folder whose
write stopped part-way has no config.json and does not load.  Reading
checks the two pairings the format encodes before any weight is used: the
drafter/ record must name the folder's weight files by their current sha256
(else `DrafterMismatch`), and tokenizer.json must hash to what every weight
header names (else `TokenizerMismatch`).  Only safetensors and JSON are read,
so loading executes nothing from the files.

The weights are this decoder's (wpt_amd.decoder.random_weights' names).  A
reference drafter/ folder holds DSpark weights with routed experts and
Attention Residuals, which this build's drafter (wpt_amd.drafter, a dense
stand-in) cannot take, so drafter/ is checked and not loaded;
`record_drafter` writes the two files the check reads.
"""

import dataclasses
import hashlib
import json
import os
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
PROVENANCE_NAME = "provenance.json"
FORMAT_ENTRY = ("format", "pt")


class DrafterMismatch(ValueError):
    """drafter/ is absent, incomplete, or names weight files other than the folder's."""


class TokenizerMismatch(ValueError):
    """tokenizer.json is absent, or is not the vocabulary the weight headers name."""


def file_sha256(path, block=1 << 20):
    """Hex sha256 of a file's bytes, streamed through one reusable buffer."""
    digest = hashlib.sha256()
    buffer = bytearray(block)
    view = memoryview(buffer)
    with open(path, "rb", buffering=0) as stream:
        while True:
            n = stream.readinto(buffer)
            if not n:
                return digest.hexdigest()
            digest.update(view[:n])


def part_names(count):
    """The file names of a weight set written in `count` parts."""
    if count == 1:
        return [SINGLE_NAME]
    return [f"model-{i:05d}-of-{count:05d}.safetensors" for i in range(1, count + 1)]


def plan_parts(sizes, limit):
    """Groups of tensor names, in order, each at most `limit` bytes unless a
    single tensor exceeds it.  sizes: {name: bytes} in the weights' order."""
    if limit is None:
        return [list(sizes)]
    groups = [[]]
    used = 0
    for name, size in sizes.items():
        if groups[-1] and used + size > limit:
            groups.append([])
            used = 0
        groups[-1].append(name)
        used += size
    return groups


def _write_json(path, value):
    staged = path.with_name(path.name + ".partial")
    staged.write_text(json.dumps(value, indent=2) + "\n", encoding="utf-8", newline="\n")
    os.replace(staged, path)


class ModelFolder:
    """One model folder on disk."""

    def __init__(self, directory):
        self.path = Path(directory)

    # -- the weight files -------------------------------------------------

    def files(self):
        """The weight file names, sorted: model.safetensors or the parts the index lists."""
        index = self.path / INDEX_NAME
        if not index.exists():
            return [SINGLE_NAME]
        mapping = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        return sorted(set(mapping.values()))

    def digests(self):
        """{weight file: sha256}, what a drafter record names."""
        return {name: file_sha256(self.path / name) for name in self.files()}

    # -- writing ----------------------------------------------------------

    def write(self, config, weights, vocabulary, vocabulary_name, shard_limit=None, header=None):
        """Replaces whatever model the directory held with `weights` (a dict
        of tensors), the vocabulary bytes and the config; config.json last."""
        self.path.mkdir(parents=True, exist_ok=True)
        for stale in [*self.path.glob("model*.safetensors"), *(self.path / n for n in
                                                                (INDEX_NAME, CONFIG_NAME, TOKENIZER_NAME))]:
            stale.unlink(missing_ok=True)
        tensors = {name: t.detach().to("cpu").contiguous() for name, t in weights.items()}
        entries = dict(header or {})
        entries["tokenizer"] = vocabulary_name
        entries["tokenizer_sha256"] = hashlib.sha256(vocabulary).hexdigest()
        entries[FORMAT_ENTRY[0]] = FORMAT_ENTRY[1]
        (self.path / TOKENIZER_NAME).write_bytes(vocabulary)
        sizes = {name: t.numel() * t.element_size() for name, t in tensors.items()}
        groups = plan_parts(sizes, shard_limit)
        names = part_names(len(groups))
        for file_name, group in zip(names, groups):
            save_file({n: tensors[n] for n in group}, self.path / file_name, metadata=entries)
        if len(groups) > 1:
            _write_json(self.path / INDEX_NAME, {
                "metadata": {"total_size": sum(sizes.values())},
                "weight_map": {n: file_name for file_name, group in zip(names, groups) for n in group}})
        _write_json(self.path / CONFIG_NAME, dataclasses.asdict(config))

    def record_drafter(self, config=None, provenance=None):
        """drafter/config.json and drafter/provenance.json; the provenance
        names the folder's current weight files unless given."""
        where = self.path / DRAFTER_NAME
        where.mkdir(parents=True, exist_ok=True)
        record = provenance if provenance is not None else {"target": {"weights": self.digests()}}
        _write_json(where / PROVENANCE_NAME, record)
        _write_json(where / CONFIG_NAME, config or {})

    # -- checks -----------------------------------------------------------

    def verify_drafter(self):
        """Raises DrafterMismatch unless drafter/ is whole and was trained
        against exactly these weight files."""
        where = self.path / DRAFTER_NAME
        record_path = where / PROVENANCE_NAME
        if not record_path.exists():
            raise DrafterMismatch(f"{self.path}: no drafter ({DRAFTER_NAME}/): the weights and the drafter "
                                  "trained against them are kept together")
        if not (where / CONFIG_NAME).exists():
            raise DrafterMismatch(f"{self.path}: its drafter ({DRAFTER_NAME}/) was not saved whole")
        record = json.loads(record_path.read_text(encoding="utf-8"))
        named = (record.get("target") or {}).get("weights")
        present = self.digests()
        if named != present:
            raise DrafterMismatch(f"{self.path}: its drafter was trained against weights {named}; the folder's "
                                  f"files are {present}")

    def vocabulary_identity(self):
        """(name, sha256) of the vocabulary, as every weight header names it."""
        named = set()
        for file_name in self.files():
            with safe_open(self.path / file_name, framework="pt") as handle:
                entries = handle.metadata() or {}
            named.add((entries.get("tokenizer"), entries.get("tokenizer_sha256")))
        (only,) = named if len(named) == 1 else (None,)
        if only is None or None in only:
            raise TokenizerMismatch(f"{self.path}: the weight headers do not agree on one named tokenizer: "
                                    f"{sorted(named, key=str)}")
        return only

    def vocabulary(self):
        """tokenizer.json's bytes, once they hash to what the weights name."""
        name, wanted = self.vocabulary_identity()
        path = self.path / TOKENIZER_NAME
        if not path.exists():
            raise TokenizerMismatch(f"{self.path}: no {TOKENIZER_NAME}; the weights name tokenizer {name}")
        data = path.read_bytes()
        found = hashlib.sha256(data).hexdigest()
        if found != wanted:
            raise TokenizerMismatch(f"{self.path}: {TOKENIZER_NAME} hashes to {found}; the weights were trained "
                                    f"with tokenizer {name} ({wanted})")
        return data

    # -- reading ----------------------------------------------------------

    def config(self):
        fields = json.loads((self.path / CONFIG_NAME).read_text(encoding="utf-8"))
        fields["kinds"] = tuple(fields.get("kinds", ()))
        return DecoderConfig(**fields)

    def weights(self):
        """(config, {name: CPU tensor}) after the drafter check."""
        self.verify_drafter()
        config = self.config()
        merged = {}
        for file_name in self.files():
            merged.update(load_file(self.path / file_name))
        return config, merged

    def decoder(self, dtype=torch.bfloat16, device="cuda"):
        """The folder's decoder on the GPU (the reference's load_model, checkpoint.py:97-107)."""
        config, weights = self.weights()
        return MQADecoder(config, weights, dtype=dtype, device=device)


# The reference's module-level names (checkpoint.py:56-169), over ModelFolder.

def save_folder(config, weights, directory, tokenizer, tokenizer_name, max_shard_bytes=None, metadata=None):
    ModelFolder(directory).write(config, weights, tokenizer, tokenizer_name, max_shard_bytes, metadata)


def save_drafter_record(directory, config=None, provenance=None):
    ModelFolder(directory).record_drafter(config, provenance)


def load_weights(directory):
    return ModelFolder(directory).weights()


def load_decoder(directory, dtype=torch.bfloat16, device="cuda"):
    return ModelFolder(directory).decoder(dtype, device)


def check_drafter(directory):
    ModelFolder(directory).verify_drafter()


def tokenizer_identity(directory):
    return ModelFolder(directory).vocabulary_identity()


def load_tokenizer(directory):
    return ModelFolder(directory).vocabulary()


def weight_files(directory):
    return ModelFolder(directory).files()


def weight_hashes(directory):
    return ModelFolder(directory).digests()
