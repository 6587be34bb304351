"""Host-side engine pieces of the FP8-V path: paged cache, cache API, accounting."""
