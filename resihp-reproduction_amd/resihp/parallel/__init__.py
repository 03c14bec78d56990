"""One TP rank's shard computation, the on-device TP re-slice and the 1F1B stage driver."""
