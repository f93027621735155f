"""The oracle: a CPU restatement of the reference's PQ search path (vk_oracle.c) and bindings to it and to the
reference's own CPU library compiled into oracle/_ref. Test infrastructure only: tests, the smoke check and the
CPU-baseline leg of bench.py use it as the checker; the product never does."""
