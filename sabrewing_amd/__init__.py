"""sabrewing_amd -- MI355X-native (gfx950 HIP) MoE block for sabrewing engines."""
