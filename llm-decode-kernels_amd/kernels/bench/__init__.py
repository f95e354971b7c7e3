"""Measurement harness: seeded cases, hipGraph timing with rotating buffers, byte accounting."""
