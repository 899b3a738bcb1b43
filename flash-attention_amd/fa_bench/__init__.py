"""Benchmark harness around flash_attention_runtime (the reference's
benchmark/ tree re-built for this library): input generation modes, the
30-column CSV schema, and the pybind benchmark CLI."""
