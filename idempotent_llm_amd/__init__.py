"""MI355X-native third backend ("rocm") for DetLLM's integer forward pass."""
