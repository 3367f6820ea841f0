"""Runtime settings mirrored from the reference (``src/sparsefold/runtime/config.py``)."""
