"""Host-side instruction API for the MI355X MoE decode megakernel.

Mirrors the reference's ``megakernels`` Python surface for the Mixtral
batch-1 MoE path (instruction dataclasses and their 32-word serialisation,
DAG scheduling, per-worker queue tensorisation, the ``interpret_with_mk``
launcher) so that callers written against the reference drive the HIP
kernel in ``csrc/mk_mixtral.hip`` unchanged.
"""
