"""MI355X-native MACE-ICTC whole-model entry points (drop-in for the reference's ``mace_ictc.hp``)."""
