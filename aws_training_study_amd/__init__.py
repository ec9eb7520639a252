"""MI355X-native history-only prefill context-parallel (PCP) attention.

``aws_training_study_amd.pcp_attention`` mirrors the ``pcp_attention``
package of the Trainium2 proof of concept (config, striped layout, kernel
entry); the device path is a hand-written gfx950 HIP kernel behind a C ABI.
"""
