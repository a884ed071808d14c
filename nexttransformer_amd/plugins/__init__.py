"""Plugin methods for the reference's plugin registry (nexttransformer/models/plugins.py:1-22).

Point NEXTTRANSFORMER_METHOD_PATHS at this directory; each subdirectory holds a method.json and
the package that defines the hooks.
"""
from pathlib import Path

ROOT = Path(__file__).resolve().parent
