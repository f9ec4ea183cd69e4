"""MI355X-native FP8 block-quantization path of pratchya's ``_qualia`` library."""
