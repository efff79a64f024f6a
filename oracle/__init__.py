"""CPU oracle of the KV-cache path (test infrastructure; never a product code path)."""
