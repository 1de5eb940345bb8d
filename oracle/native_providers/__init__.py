"""Native (pure-PyTorch, CPU) providers restating the reference's native ops.

Attach them to a dispatcher with
``torchturbo_amd.dispatch.add_provider_package("oracle.native_providers")``.
Test infrastructure only.
"""
