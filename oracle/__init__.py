"""ORACLE: the CPU restatement the HIP path is tested against. Test infrastructure only; the product never imports it."""
