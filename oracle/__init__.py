"""CPU oracle of the reshard repack -- test infrastructure only.

Nothing here is part of the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
it, and only to check results against (or as the timed CPU restatement
of the reference); the product path never routes through it.

Contents
  synth          numpy restatement of the seeded synthetic generator
  synth_ref.c    C restatement of the same generator (cross-check)
  model          parameter inventory of a model (names, shapes, TP attributes)
  megatron_buffer  Megatron-core DDP buffer layout rules
  plan           the reference's per-parameter plan: TP send/recv maps
                 (resharding_tp.py:94-191), stages (resharding_pp.py:96-122),
                 expert ranks (resharding_dp.py:21-34), DP distributions
                 (resharding_dp.py:224-409), global ranks (resharding.py:19-51),
                 aligned ranks and global send/recv maps (resharding.py:54-162)
  transfer       Oracle-1: the reference's three-pass executor
                 (transfer/transfer.py:36-341) with a FIFO mailbox standing in
                 for send/recv and self copies (communicator.py:38-96), the
                 SwiGLU shuffle (resharding_metadata.py:98-178), the bf16
                 rebuild (training_state.py:176-197) and Group-ZeRO backup
                 (transfer.py:343-388, training_state.py:40-60)
  canonical      Oracle-2: every destination piece regenerated from its
                 full-tensor indices, independent of any plan

Parity status
  megatron_buffer: parity unpinned.  Megatron-core (core_r0.11.0) is not
  vendored with the reference and cannot be imported here; its layout rules
  are restated from its published algorithm and checked by invariants and by
  known answers derived by hand from that algorithm for every branch
  (reverse order, start and end padding, the >= bucket close, shared
  embeddings, expert buffers; tests/test_ddp_layout.py), never against
  Megatron itself.
  canonical.world(vocab_rows=...): the vocabulary re-padding extension has
  no counterpart in the reference (virtual_param.py:480-481 keeps the padded
  vocabulary fixed); it is an invariant (kept rows keep their values, new
  rows are zero), checked by grow-then-shrink round trips.
  Every other function is pinned by closed forms, brute force on small
  shapes, or the Oracle-1 == Oracle-2 cross-check (see tests/).
"""
