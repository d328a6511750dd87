"""ORACLE: the CPU checker for the HIP path. Test infrastructure only; the product never imports it."""
