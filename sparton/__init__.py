"""Drop-in import name of the reference package: `from sparton import SpartonHead`
(training/model.py:72, README.md:21) resolves to the MI355X implementation."""
from sparton_amd import SpartonHead

__all__ = ["SpartonHead"]
