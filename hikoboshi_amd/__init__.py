"""MI355X-native ProteinMPNN v_48_020 design path (HIP/CDNA4)."""
