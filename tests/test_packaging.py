"""Plugin registration in package metadata (the reference's pyproject.toml:12-13).

vLLM finds general plugins through the ``vllm.general_plugins`` entry-point group and
calls each target once per process.  These tests read this repository's
pyproject.toml, resolve the declared target the way importlib.metadata does, and check
that it is the plugin's idempotent, argument-free ``load_plugin``.
"""
from importlib.metadata import EntryPoint
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

try:
    import tomllib as toml_reader
except ModuleNotFoundError:  # Python 3.10
    import tomli as toml_reader


@pytest.fixture(scope="module")
def project():
    return toml_reader.loads((ROOT / "pyproject.toml").read_text())


def test_general_plugin_entry_point_resolves_to_load_plugin(project):
    from oscar_amd import plugin

    group = project["project"]["entry-points"]["vllm.general_plugins"]
    assert group == {"oscar_amd": "oscar_amd.plugin:load_plugin"}
    target = EntryPoint(name="oscar_amd", value=group["oscar_amd"], group="vllm.general_plugins").load()
    assert target is plugin.load_plugin
    import inspect

    assert not inspect.signature(target).parameters  # vLLM calls it with no arguments


def test_package_discovery_finds_the_package_and_its_library(project):
    from setuptools import find_packages

    find = project["tool"]["setuptools"]["packages"]["find"]
    found = find_packages(where=str(ROOT / find["where"][0] if isinstance(find["where"], list) else ROOT),
                          include=find["include"])
    assert "oscar_amd" in found and not any(p.startswith(("tests", "oracle")) for p in found)
    data = project["tool"]["setuptools"]["package-data"]["oscar_amd"]
    assert "liboscar_amd.so" in data  # the C ABI the package loads (oscar_amd/_lib.py)
    assert project["project"]["name"] and project["project"]["requires-python"] == ">=3.10"
