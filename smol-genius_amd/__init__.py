"""MI355X-native attention path for smol-genius (HIP for gfx950 behind a C ABI)."""
