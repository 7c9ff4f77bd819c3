"""Dense (Llama) low-latency VM: globals, instruction set, scheduler and
launcher (counterpart of ``megakernels/demos/latency/``)."""
