"""Reload errors of the layer file reader (serialization.py), raised before
any GPU work (tests/test_serialization.py:187-196 of the reference)."""

from __future__ import annotations

import pytest

from exl3_intel_arc_quantizer_amd.serialization import load_and_verify_layer_safetensors


def test_missing_file_raises(tmp_path):
    with pytest.raises(FileNotFoundError):
        load_and_verify_layer_safetensors(tmp_path / "nonexistent.safetensors")


def test_truncated_file_raises(tmp_path):
    bad = tmp_path / "truncated.safetensors"
    bad.write_bytes(b"\x00\x00\x00\x00badheader")
    with pytest.raises(Exception):
        load_and_verify_layer_safetensors(bad)
