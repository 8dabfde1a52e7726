"""ctypes binding of libeoship.so (declared in include/eoship.h).

The library is the only compute path: when it is missing or fails to load,
every call raises; there is no host fallback.
"""
from __future__ import annotations

import ctypes as C
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libeoship.so")

c_err = C.POINTER(C.c_char_p)


class EosHipTQDesc(C.Structure):
    _fields_ = [
        ("dim", C.c_int32),
        ("bits", C.c_int32),
        ("codebook_scale", C.c_float),
        ("codebook", C.POINTER(C.c_int8)),
        ("rotation", C.POINTER(C.c_float)),
    ]


class EosHipTQBindOptions(C.Structure):
    _fields_ = [
        ("zero_vector_allowed", C.POINTER(C.c_uint8)),
        ("id_rank", C.POINTER(C.c_int64)),
    ]


class EosHipTQStats(C.Structure):
    _fields_ = [
        ("candidate_count", C.c_int64),
        ("candidates_kept", C.c_int64),
        ("fallback_queries", C.c_int32),
        ("batches", C.c_int32),
    ]


class EosHipEncoderDesc(C.Structure):
    _fields_ = [
        ("layers", C.c_int32),
        ("hidden", C.c_int32),
        ("heads", C.c_int32),
        ("intermediate", C.c_int32),
        ("vocab", C.c_int32),
        ("max_positions", C.c_int32),
        ("type_vocab", C.c_int32),
        ("ln_eps", C.c_float),
        ("gelu", C.c_int32),
    ]


_I8P = C.POINTER(C.c_int8)
_F32P = C.POINTER(C.c_float)


class EosHipEncoderLayer(C.Structure):
    _fields_ = [
        ("w_qkv", _I8P), ("s_qkv", _F32P), ("b_qkv", _F32P),
        ("w_o", _I8P), ("s_o", _F32P), ("b_o", _F32P),
        ("ln1_gamma", _F32P), ("ln1_beta", _F32P),
        ("w_1", _I8P), ("s_1", _F32P), ("b_1", _F32P),
        ("w_2", _I8P), ("s_2", _F32P), ("b_2", _F32P),
        ("ln2_gamma", _F32P), ("ln2_beta", _F32P),
    ]


class EosHipCompactDesc(C.Structure):
    _fields_ = [
        ("layers", C.c_int32),
        ("model_dim", C.c_int32),
        ("heads", C.c_int32),
        ("hidden_dim", C.c_int32),
        ("vocab", C.c_int32),
        ("max_sequence", C.c_int32),
        ("output_dim", C.c_int32),
    ]


class EosHipCompactLayer(C.Structure):
    _fields_ = [
        ("attn_q", _I8P), ("s_q", C.c_float),
        ("attn_k", _I8P), ("s_k", C.c_float),
        ("attn_v", _I8P), ("s_v", C.c_float),
        ("attn_o", _I8P), ("s_o", C.c_float),
        ("ffn_up", _I8P), ("s_up", C.c_float),
        ("ffn_down", _I8P), ("s_down", C.c_float),
    ]


class EosHipCompactOptions(C.Structure):
    _fields_ = [
        ("rope", C.c_int32),
        ("role", C.c_int32),
        ("scaled_scores", C.c_int32),
        ("attend_padding", C.c_int32),
    ]


class EosHipMllInfo(C.Structure):
    _fields_ = [
        ("profile", C.c_int32),
        ("sections", C.c_int32),
        ("strings", C.c_int64),
        ("tensors", C.c_int64),
        ("has_metadata", C.c_int32),
        ("module_name", C.c_char * 128),
        ("module_version", C.c_char * 64),
    ]


class EosHipMllTensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("kind", C.c_int32),
        ("storage_dtype", C.c_int32),
        ("rank", C.c_int32),
        ("dims", C.c_int64 * 8),
        ("elements", C.c_int64),
        ("data", C.c_void_p),
        ("bytes", C.c_uint64),
        ("scale", C.c_float),
    ]


class EosHipAccounting(C.Structure):
    _fields_ = [
        ("kernel_launches", C.c_int64),
        ("uploaded_bytes", C.c_int64),
        ("downloaded_bytes", C.c_int64),
        ("sync_count", C.c_int64),
        ("graph_captures", C.c_int64),
        ("graph_replays", C.c_int64),
        ("device_execution", C.c_int32),
        ("reserved", C.c_int32),
    ]


class EosHipMllPlan(C.Structure):
    _fields_ = [
        ("route", C.c_int32),
        ("layers", C.c_int32),
        ("distinct_layers", C.c_int32),
        ("model_dim", C.c_int32),
        ("heads", C.c_int32),
        ("hidden_dim", C.c_int32),
        ("vocab", C.c_int32),
        ("max_sequence", C.c_int32),
        ("output_dim", C.c_int32),
        ("batched", C.c_int32),
        ("steps", C.c_int32),
        ("options", EosHipCompactOptions),
        ("entry", C.c_char * 64),
        ("token_input", C.c_char * 64),
        ("mask_input", C.c_char * 64),
        ("output_name", C.c_char * 64),
        ("pooling", C.c_int32),
        ("type_vocab", C.c_int32),
        ("weights_quantized", C.c_int32),
        ("reserved", C.c_int32),
        ("ln_eps", C.c_double),
        ("type_input", C.c_char * 64),
    ]


class EosHipScoreSpec(C.Structure):
    _fields_ = [
        ("op", C.c_int32),
        ("k", C.c_int32),
        ("docs_q4", C.c_int32),
        ("docs_scale", C.c_float),
        ("batched", C.c_int32),
    ]


class EosHipRetrievalPlan(C.Structure):
    _fields_ = [
        ("op", C.c_int32),
        ("k", C.c_int32),
        ("batched", C.c_int32),
        ("docs_param", C.c_int32),
        ("has_candidate_ids", C.c_int32),
        ("docs_q4", C.c_int32),
        ("docs_rows", C.c_int64),
        ("dim", C.c_int32),
        ("n_outputs", C.c_int32),
        ("outputs", C.c_int32 * 8),
        ("steps", C.c_int32),
        ("entry", C.c_char * 64),
        ("query_input", C.c_char * 64),
        ("docs_input", C.c_char * 64),
        ("ids_input", C.c_char * 64),
    ]


class EosHipTQCodes(C.Structure):
    _fields_ = [
        ("bits", C.c_int32),
        ("dim", C.c_int32),
        ("n", C.c_int64),
        ("codes", C.c_void_p),
        ("norms", C.c_void_p),
        ("codebook", C.c_void_p),
        ("rotation_t", C.c_void_p),
        ("signs", C.c_void_p),
        ("resnorms", C.c_void_p),
        ("qjl_t", C.c_void_p),
    ]


class EosHipHadamardSpec(C.Structure):
    _fields_ = [
        ("channels", C.c_int32),
        ("bits", C.c_int32),
        ("perm", C.c_void_p),
        ("signs1", C.c_void_p),
        ("signs2", C.c_void_p),
        ("centroids", C.c_void_p),
        ("boundaries", C.c_void_p),
    ]


class EosHipTQIPSpec(C.Structure):
    _fields_ = [
        ("dim", C.c_int32),
        ("bits", C.c_int32),
        ("codebook_scale", C.c_float),
        ("codebook", C.c_void_p),
        ("rotation_t", C.c_void_p),
        ("qjl_t", C.c_void_p),
    ]


# name -> (argtypes) ; every function returns int except where noted
_SIGNATURES = {
    "eoship_abi_version": ([], C.c_int),
    "eoship_free_cstring": ([C.c_void_p], None),
    "eoship_runtime_create": ([C.c_int, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_runtime_destroy": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_device_info": ([C.c_void_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_int), C.c_char_p,
                            C.c_size_t, C.c_void_p], C.c_int),
    "eoship_malloc": ([C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_free": ([C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_h2d": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "eoship_d2h": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "eoship_d2d": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "eoship_accounting_read": ([C.c_void_p, C.POINTER(EosHipAccounting), C.c_int32, C.c_void_p],
                               C.c_int),
    "eoship_memset": ([C.c_void_p, C.c_void_p, C.c_int, C.c_size_t, C.c_void_p], C.c_int),
    "eoship_sync": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_runtime_wait": ([C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_module_load": ([C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p), C.c_void_p],
                           C.c_int),
    "eoship_module_unload": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_function": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_launch": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                       C.c_uint32, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_profile_enable": ([C.c_void_p, C.c_int, C.c_void_p], C.c_int),
    "eoship_profile_select": ([C.c_void_p, C.c_char_p, C.c_void_p], C.c_int),
    "eoship_profile_read": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_int64), C.POINTER(C.c_double),
                             C.c_void_p], C.c_int),
    "eoship_profile_reset": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_profile_samples": ([C.c_void_p, C.c_char_p, C.c_void_p, C.c_int64,
                                C.POINTER(C.c_int64), C.c_void_p], C.c_int),
    "eoship_timer_mark": ([C.c_void_p, C.c_int, C.c_void_p], C.c_int),
    "eoship_timer_elapsed": ([C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_double), C.c_void_p],
                             C.c_int),
    "eoship_tq_bind_corpus": ([C.c_void_p, C.POINTER(EosHipTQDesc), C.c_void_p, C.c_void_p,
                               C.c_int64, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_tq_bind_corpus_opts": ([C.c_void_p, C.POINTER(EosHipTQDesc), C.c_void_p, C.c_void_p,
                                    C.c_int64, C.POINTER(EosHipTQBindOptions),
                                    C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_tq_vector_bytes": ([C.c_int32, C.c_int32, C.POINTER(C.c_int64), C.c_void_p], C.c_int),
    "eoship_tq_mse_vector_bytes": ([C.c_int32, C.c_int32, C.POINTER(C.c_int64), C.c_void_p],
                                   C.c_int),
    "eoship_tq_release": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_share": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_tq_topk": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                        C.c_void_p, C.POINTER(EosHipTQStats), C.c_void_p], C.c_int),
    "eoship_tq_topk_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                               C.c_void_p, C.c_void_p, C.POINTER(EosHipTQStats), C.c_void_p],
                              C.c_int),
    "eoship_tq_topk_device_deferred": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_topk_repair_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_scores": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int64, C.c_int64,
                          C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_prepare": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                           C.c_void_p], C.c_int),
    "eoship_tq_maxsim_topk": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int32,
                               C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_maxsim_topk_device": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32,
                                      C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p],
                                     C.c_int),
    "eoship_tq_maxsim_scores": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int32,
                                 C.c_int64, C.c_int64, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_f16_sidecar_device": ([C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_fp16_rerank_device": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                                      C.c_int64, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                      C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p], C.c_int),
    "eoship_tq_fp16_rerank_device_noalloc": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                              C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                                              C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                              C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p],
                                             C.c_int),
    "eoship_tq_encode": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                          C.c_void_p], C.c_int),
    "eoship_tq_encode_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p,
                                 C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_parents_bind": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_tq_parents_release": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_parent_topk": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                               C.c_double, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                               C.c_void_p], C.c_int),
    "eoship_tq_parent_topk_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                      C.c_int32, C.c_double, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p], C.c_int),
    "eoship_embed_bind": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_int32,
                           C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_embed_release": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_embed_run": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p],
                         C.c_int),
    "eoship_embed_run_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                 C.c_void_p], C.c_int),
    "eoship_encoder_bind": ([C.c_void_p, C.POINTER(EosHipEncoderDesc), _F32P, _F32P, _F32P, _F32P,
                             _F32P, C.POINTER(EosHipEncoderLayer), C.POINTER(C.c_void_p),
                             C.c_void_p], C.c_int),
    "eoship_encoder_bind_compact": ([C.c_void_p, C.POINTER(EosHipCompactDesc), _I8P, C.c_float,
                                     _I8P, C.c_float, C.POINTER(EosHipCompactLayer), _I8P,
                                     C.c_float, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_encoder_bind_compact_opts": ([C.c_void_p, C.POINTER(EosHipCompactDesc),
                                          C.POINTER(EosHipCompactOptions), _I8P, C.c_float, _I8P,
                                          C.c_float, C.POINTER(EosHipCompactLayer), _I8P,
                                          C.c_float, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_mll_open": ([C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p), C.c_void_p], C.c_int),
    "eoship_mll_close": ([C.c_void_p], None),
    "eoship_mll_info": ([C.c_void_p, C.POINTER(EosHipMllInfo), C.c_void_p], C.c_int),
    "eoship_mll_section": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p),
                            C.POINTER(C.c_uint64), C.c_void_p], C.c_int),
    "eoship_mll_tensor": ([C.c_void_p, C.c_int64, C.c_char_p, C.POINTER(EosHipMllTensor),
                           C.c_void_p], C.c_int),
    "eoship_blake3": ([C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_mll_classify": ([C.c_void_p, C.c_char_p, C.POINTER(EosHipMllPlan), C.c_void_p],
                            C.c_int),
    "eoship_encoder_bind_mll": ([C.c_void_p, C.c_void_p, C.c_char_p, C.c_int32,
                                 C.POINTER(C.c_void_p), C.POINTER(EosHipMllPlan), C.c_void_p],
                                C.c_int),
    "eoship_score_topk_device": ([C.c_void_p, C.POINTER(EosHipScoreSpec), C.c_void_p, C.c_int32,
                                  C.c_int32, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                                  C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p],
                                 C.c_int),
    "eoship_mll_classify_retrieval": ([C.c_void_p, C.c_char_p, C.POINTER(EosHipRetrievalPlan),
                                       C.c_void_p], C.c_int),
    "eoship_retrieval_bind_mll": ([C.c_void_p, C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p),
                                   C.POINTER(EosHipRetrievalPlan), C.c_void_p], C.c_int),
    "eoship_retrieval_run_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                     C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_retrieval_release": ([C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_dense_rerank_device": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                                       C.c_int64, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_reconstruct_rerank_device": ([C.c_void_p, C.POINTER(EosHipTQCodes), C.c_void_p,
                                             C.c_int32, C.c_void_p, C.c_int32, C.c_int32,
                                             C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p],
                                            C.c_int),
    "eoship_hadamard_tq_bind": ([C.c_void_p, C.POINTER(EosHipHadamardSpec), C.POINTER(C.c_void_p),
                                 C.c_void_p], C.c_int),
    "eoship_hadamard_tq_encode_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                                          C.c_int32, C.c_int32, C.c_void_p, C.c_void_p,
                                          C.c_void_p], C.c_int),
    "eoship_hadamard_tq_decode_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                          C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                          C.c_void_p], C.c_int),
    "eoship_hadamard_tq_release": ([C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_ip_encode_device": ([C.c_void_p, C.POINTER(EosHipTQIPSpec), C.c_void_p, C.c_int64,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p],
                                   C.c_int),
    "eoship_tq_ip_bind_corpus": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                  C.c_void_p, C.c_int64, C.c_void_p, C.POINTER(C.c_void_p),
                                  C.c_void_p], C.c_int),
    "eoship_tq_ip_topk_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                  C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_ip_release": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_tq_ip_scores_device": ([C.c_void_p, C.POINTER(EosHipTQIPSpec), C.c_void_p, C.c_int32,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                    C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p],
                                   C.c_int),
    "eoship_encoder_release": ([C.c_void_p, C.c_void_p], C.c_int),
    "eoship_encoder_forward": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.c_int32, C.c_int32, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_encoder_forward_device": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_int32, C.c_int32, C.c_void_p, C.c_void_p], C.c_int),
    "eoship_encoder_status": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_int32), C.c_void_p], C.c_int),
    "eoship_encoder_set_fused_tail": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p], C.c_int),
    "eoship_encoder_set_pooling": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p], C.c_int),
    "eoship_encoder_attention_moves": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_int64), C.c_void_p],
                                       C.c_int),
}

_lib = None


class EosHipError(RuntimeError):
    """Error reported by libeoship (the char** err message)."""


def load() -> C.CDLL:
    """Load libeoship.so and declare its prototypes; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise EosHipError(
            f"{LIB_PATH} is not built; run `python -m eos_amd.build` (the HIP library is the only "
            "compute path)")
    lib = C.CDLL(LIB_PATH)
    for name, (argtypes, restype) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def call(name: str, *args) -> None:
    """Call an int-returning entry point with a trailing char** err; raise on failure."""
    lib = load()
    err = C.c_char_p()
    rc = getattr(lib, name)(*args, C.byref(err))
    if rc != 0:
        msg = err.value.decode("utf-8", "replace") if err.value else f"{name} failed"
        if err.value:
            lib.eoship_free_cstring(C.cast(err, C.c_void_p))
        raise EosHipError(msg)
