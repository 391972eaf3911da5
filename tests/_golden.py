"""Loader for the golden vectors written by tests/golden/make_golden.py."""

import json
import os

from safetensors.torch import load_file

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def index():
    with open(os.path.join(GOLDEN, "index.json")) as f:
        return json.load(f)


def load(name):
    meta = index()[name]
    return load_file(os.path.join(GOLDEN, f"{name}.safetensors")), meta


def names(kind=None):
    return sorted(n for n, m in index().items() if kind is None or m["kind"] == kind)


def producer_index():
    with open(os.path.join(GOLDEN, "producer_index.json")) as f:
        return json.load(f)


def load_producer(name):
    """A key-producer case written by tests/golden/make_producer_golden.py."""
    meta = producer_index()[name]
    return load_file(os.path.join(GOLDEN, f"{name}.safetensors")), meta


def producer_names(kind=None):
    return sorted(n for n, m in producer_index().items() if kind is None or m["kind"] == kind)
