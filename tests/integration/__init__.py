"""The reference-side bindings of the integration guide, as runnable files."""
