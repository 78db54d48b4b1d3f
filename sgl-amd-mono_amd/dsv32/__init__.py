"""The DeepSeek-V3.2-geometry DSA layer on gfx950: geometry, host ops and the spec."""
