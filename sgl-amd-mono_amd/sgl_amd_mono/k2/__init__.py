"""The K2 decode layer on MI355X: configs, encoders, tile packing, host ops, spec."""
