"""Host side of the MI355X batch-1 decode kernels: op loader (``ext``), INT4 weight format (``quant``), synthetic
Llama weights (``synth``) and the graph-captured decode runtime (``model``). Mirrors the reference's ``runtime``
package so call sites read the same (``from runtime import ext``; ``K = ext.load()``)."""
