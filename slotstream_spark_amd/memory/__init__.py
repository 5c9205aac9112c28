"""Expert slot pool in HBM: record layout, map / slot_ptr tables, synthetic records."""
