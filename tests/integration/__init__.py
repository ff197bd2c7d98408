"""The reference-side bindings shown in INTEGRATION.md, as runnable files."""
