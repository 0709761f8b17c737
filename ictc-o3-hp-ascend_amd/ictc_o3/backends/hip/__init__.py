"""HIP backend: autograd schedules over libictc_hip.so."""
