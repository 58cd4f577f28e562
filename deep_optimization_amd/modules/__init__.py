"""Host-side mirror of Activation_Compression/modules: group layout and quantize plumbing."""
