"""korith_vllm_ext - MI355X (gfx950) implementation of Axropus AMF's KV
materialization path, keeping the reference package's module paths and APIs
(CompressedVRAMPool, AmfKvManager / AmfKVManager, AmfWorkerExtension,
int4_decode_attention, the codec registry).  Device work runs in
libamf_hip.so through the ctypes binding in amf_hip/."""
