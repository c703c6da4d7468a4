"""TEST INFRASTRUCTURE ONLY: the CPU oracle of the static INT8 KV-cache path.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg -- never by the product
package (int8-kvcache_amd/kvq)."""
