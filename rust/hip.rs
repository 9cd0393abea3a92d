//! HIP (AMD Instinct MI355X, gfx950) backend with the `MetalContext` surface.
//!
//! A DiskMule maintainer adds this file as `src/hip.rs` behind a cargo feature
//! `hip`. `src/metal.rs` then re-exports `MetalContext`, `MetalMappedBuffer`,
//! `MetalOwnedBuffer` and `MetalKvLayer` from here, and `src/expert.rs`
//! re-exports `ExpertCache`, so the graphs' `use crate::metal::...` and
//! `use crate::expert::...` lines compile unchanged. The types, method names,
//! argument meanings, check order and error variants are those of
//! src/metal.rs:180-1604 and src/expert.rs:64-164.
//!
//! Everything here is a thin, safe layer over `libdmhip.so` (declared in
//! `include/dmhip.h`); the arithmetic runs in that library's HIP kernels.
//! The module uses only `std` plus the crate's own `memmap2` (the `Arc<Mmap>`
//! that `map_read_only` receives).
//!
//! Status: this file is not compiled in the repository that holds it (its
//! build image has no Rust toolchain). The C ABI it binds is compiled and
//! tested there, through ctypes, with the same call sequences.

#![allow(clippy::too_many_arguments)]

use std::{
    ffi::{CStr, c_char, c_int},
    fmt, io,
    os::fd::AsRawFd,
    fs::File,
    ptr::{self, NonNull},
    rc::Rc,
    sync::Arc,
    time::Duration,
};

use memmap2::Mmap;

use crate::{
    expert::{ExpertCacheError, ExpertCacheStats, ExpertLayerLayout},
    gguf::TensorType,
    metal::MetalError,
    safetensors::SafeDtype,
};

/// One-to-one transcription of `include/dmhip.h`.
#[allow(non_camel_case_types, dead_code)]
pub mod ffi {
    use std::ffi::{c_char, c_int, c_void};

    #[repr(C)]
    pub struct dmhip_ctx {
        _opaque: [u8; 0],
    }
    #[repr(C)]
    pub struct dmhip_buf {
        _opaque: [u8; 0],
    }
    #[repr(C)]
    pub struct dmhip_expert_cache {
        _opaque: [u8; 0],
    }
    #[repr(C)]
    pub struct dmhip_kv_layer {
        _opaque: [u8; 0],
    }

    pub const DMHIP_OK: c_int = 0;
    pub const DMHIP_ERR_NO_DEVICE: c_int = 1;
    pub const DMHIP_ERR_BUFFER_ALLOCATION: c_int = 2;
    pub const DMHIP_ERR_VECTOR_LENGTH: c_int = 3;
    pub const DMHIP_ERR_VECTOR_TOO_LARGE: c_int = 4;
    pub const DMHIP_ERR_EMPTY_INPUT: c_int = 5;
    pub const DMHIP_ERR_INVALID_VECTOR_LENGTH: c_int = 6;
    pub const DMHIP_ERR_INVALID_POSITIVE_PARAMETER: c_int = 7;
    pub const DMHIP_ERR_NON_FINITE: c_int = 8;
    pub const DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE: c_int = 9;
    pub const DMHIP_ERR_INVALID_ELEMENT_COUNT: c_int = 10;
    pub const DMHIP_ERR_INVALID_BYTE_LENGTH: c_int = 11;
    pub const DMHIP_ERR_OVERFLOW: c_int = 12;
    pub const DMHIP_ERR_INVALID_INPUT_LENGTH: c_int = 13;
    pub const DMHIP_ERR_INVALID_OUTPUT_LENGTH: c_int = 14;
    pub const DMHIP_ERR_INVALID_TOP_K: c_int = 15;
    pub const DMHIP_ERR_MAPPED_RANGE: c_int = 16;
    pub const DMHIP_ERR_COMMAND: c_int = 17;
    pub const DMHIP_ERR_NO_SLOTS: c_int = 18;
    pub const DMHIP_ERR_INVALID_LAYER: c_int = 19;
    pub const DMHIP_ERR_INVALID_EXPERT: c_int = 20;
    pub const DMHIP_ERR_ALL_SLOTS_PINNED: c_int = 21;
    pub const DMHIP_ERR_CANCELLED: c_int = 22;
    pub const DMHIP_ERR_INVALID_LAYOUT: c_int = 23;
    pub const DMHIP_ERR_INVALID_ARGUMENT: c_int = 24;
    pub const DMHIP_ERR_IO: c_int = 25;
    pub const DMHIP_ERR_INVALID_ATTENTION_SHAPE: c_int = 26;
    pub const DMHIP_ERR_KV_POSITION: c_int = 27;
    pub const DMHIP_ERR_KV_WIDTH: c_int = 28;
    pub const DMHIP_ERR_KV_CONTEXT: c_int = 29;
    pub const DMHIP_ERR_INVALID_ROPE_SHAPE: c_int = 30;
    pub const DMHIP_ERR_INVALID_ROPE_PAIRS: c_int = 31;

    #[repr(C)]
    #[derive(Clone, Copy)]
    pub struct dmhip_error_detail {
        pub status: i32,
        pub os_error: i32,
        pub operation: *const c_char,
        pub argument: *const c_char,
        pub kind: *const c_char,
        pub expected: u64,
        pub actual: u64,
        pub offset: u64,
        pub end: u64,
        pub length: u64,
        pub left: u64,
        pub right: u64,
        pub output: u64,
        pub elements: u64,
        pub block_elements: u64,
        pub k: u64,
        pub bytes: u64,
        pub layer: u64,
        pub expert: u64,
        pub count: u64,
        pub position: u64,
        pub limit: u64,
        pub reason: *const c_char,
        pub heads: u64,
        pub head_dimension: u64,
    }

    impl dmhip_error_detail {
        pub fn empty() -> Self {
            Self {
                status: 0,
                os_error: 0,
                operation: std::ptr::null(),
                argument: std::ptr::null(),
                kind: std::ptr::null(),
                expected: 0,
                actual: 0,
                offset: 0,
                end: 0,
                length: 0,
                left: 0,
                right: 0,
                output: 0,
                elements: 0,
                block_elements: 0,
                k: 0,
                bytes: 0,
                layer: 0,
                expert: 0,
                count: 0,
                position: 0,
                limit: 0,
                reason: std::ptr::null(),
                heads: 0,
                head_dimension: 0,
            }
        }
    }

    #[repr(C)]
    #[derive(Clone, Copy)]
    pub struct dmhip_expert_layer_layout {
        pub expert_count: usize,
        pub gate_up_offset: u64,
        pub gate_up_bytes: usize,
        pub down_offset: u64,
        pub down_bytes: usize,
    }

    #[repr(C)]
    #[derive(Clone, Copy, Default)]
    pub struct dmhip_expert_cache_stats {
        pub hits: u64,
        pub misses: u64,
        pub evictions: u64,
        pub reads: u64,
        pub bytes_read: u64,
        pub io_wait_ns: u64,
        pub resident_bytes: u64,
    }

    pub const DMHIP_TYPE_F32: u32 = 0;
    pub const DMHIP_TYPE_F16: u32 = 1;
    pub const DMHIP_TYPE_Q5_0: u32 = 6;
    pub const DMHIP_TYPE_Q8_0: u32 = 8;
    pub const DMHIP_TYPE_Q4_K: u32 = 12;
    pub const DMHIP_TYPE_Q6_K: u32 = 14;
    pub const DMHIP_TYPE_BF16: u32 = 30;

    pub const DMHIP_SAFE_BOOL: u32 = 0;
    pub const DMHIP_SAFE_U8: u32 = 1;
    pub const DMHIP_SAFE_I8: u32 = 2;
    pub const DMHIP_SAFE_U16: u32 = 3;
    pub const DMHIP_SAFE_I16: u32 = 4;
    pub const DMHIP_SAFE_F16: u32 = 5;
    pub const DMHIP_SAFE_BF16: u32 = 6;
    pub const DMHIP_SAFE_U32: u32 = 7;
    pub const DMHIP_SAFE_I32: u32 = 8;
    pub const DMHIP_SAFE_F32: u32 = 9;
    pub const DMHIP_SAFE_U64: u32 = 10;
    pub const DMHIP_SAFE_I64: u32 = 11;
    pub const DMHIP_SAFE_F64: u32 = 12;
    pub const DMHIP_SAFE_F8_E4M3: u32 = 13;
    pub const DMHIP_SAFE_F8_E5M2: u32 = 14;

    #[link(name = "dmhip")]
    unsafe extern "C" {
        // context, errors, device
        pub fn dmhip_last_error() -> *const c_char;
        pub fn dmhip_last_error_detail(out: *mut dmhip_error_detail) -> c_int;
        pub fn dmhip_context_new(device: c_int, out: *mut *mut dmhip_ctx) -> c_int;
        pub fn dmhip_context_free(ctx: *mut dmhip_ctx);
        pub fn dmhip_device_name(ctx: *mut dmhip_ctx, buffer: *mut c_char, capacity: usize) -> c_int;
        pub fn dmhip_synchronize(ctx: *mut dmhip_ctx) -> c_int;
        pub fn dmhip_stream(ctx: *mut dmhip_ctx) -> *mut c_void;

        // buffers
        pub fn dmhip_map_read_only(
            ctx: *mut dmhip_ctx,
            host: *const c_void,
            length: usize,
            out: *mut *mut dmhip_buf,
        ) -> c_int;
        pub fn dmhip_new_owned_buffer(ctx: *mut dmhip_ctx, length: usize, out: *mut *mut dmhip_buf) -> c_int;
        pub fn dmhip_buffer_free(buffer: *mut dmhip_buf);
        pub fn dmhip_buffer_len(buffer: *const dmhip_buf) -> usize;
        pub fn dmhip_buffer_device_ptr(buffer: *const dmhip_buf) -> *mut c_void;
        pub fn dmhip_buffer_write(
            ctx: *mut dmhip_ctx,
            buffer: *mut dmhip_buf,
            offset: usize,
            src: *const c_void,
            n: usize,
        ) -> c_int;
        pub fn dmhip_buffer_read(
            ctx: *mut dmhip_ctx,
            buffer: *const dmhip_buf,
            offset: usize,
            dst: *mut c_void,
            n: usize,
        ) -> c_int;
        pub fn dmhip_copy_to_host(ctx: *mut dmhip_ctx, dst: *mut c_void, device_src: *const c_void, n: usize) -> c_int;
        pub fn dmhip_copy_to_device(ctx: *mut dmhip_ctx, device_dst: *mut c_void, src: *const c_void, n: usize)
        -> c_int;
        pub fn dmhip_host_alloc_pinned(bytes: usize, out: *mut *mut c_void) -> c_int;
        pub fn dmhip_host_free_pinned(ptr: *mut c_void);

        // synchronous host-slice operators
        pub fn dmhip_rms_norm(
            ctx: *mut dmhip_ctx,
            input: *const f32,
            input_len: usize,
            weight: *const f32,
            weight_len: usize,
            epsilon: f32,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_silu_mul(
            ctx: *mut dmhip_ctx,
            gate: *const f32,
            gate_len: usize,
            up: *const f32,
            up_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_softcap(
            ctx: *mut dmhip_ctx,
            input: *const f32,
            input_len: usize,
            cap: f32,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_add(
            ctx: *mut dmhip_ctx,
            left: *const f32,
            left_len: usize,
            right: *const f32,
            right_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_gelu_mul(
            ctx: *mut dmhip_ctx,
            gate: *const f32,
            gate_len: usize,
            up: *const f32,
            up_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_softmax(
            ctx: *mut dmhip_ctx,
            input: *const f32,
            input_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_rope_neox_in_place(
            ctx: *mut dmhip_ctx,
            values: *mut f32,
            values_len: usize,
            heads: usize,
            head_dimension: usize,
            rotated_pairs: usize,
            position: usize,
            theta: f32,
        ) -> c_int;
        pub fn dmhip_add_device(
            ctx: *mut dmhip_ctx,
            count: usize,
            left: *const f32,
            right: *const f32,
            output: *mut f32,
        ) -> c_int;
        pub fn dmhip_gelu_mul_device(
            ctx: *mut dmhip_ctx,
            count: usize,
            gate: *const f32,
            up: *const f32,
            output: *mut f32,
        ) -> c_int;
        pub fn dmhip_rope_neox_device(
            ctx: *mut dmhip_ctx,
            values: *mut f32,
            values_len: usize,
            heads: usize,
            head_dimension: usize,
            rotated_pairs: usize,
            position: usize,
            theta: f32,
        ) -> c_int;
        pub fn dmhip_argmax(ctx: *mut dmhip_ctx, input: *const f32, input_len: usize, index: *mut usize) -> c_int;
        pub fn dmhip_top_k_softmax(
            ctx: *mut dmhip_ctx,
            logits: *const f32,
            logits_len: usize,
            k: usize,
            indices: *mut usize,
            probabilities: *mut f32,
        ) -> c_int;
        pub fn dmhip_matvec(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            rows: usize,
            columns: usize,
            encoded: *const u8,
            encoded_len: usize,
            input: *const f32,
            input_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_matvec_mapped(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            rows: usize,
            columns: usize,
            mapping: *const dmhip_buf,
            encoded_offset: usize,
            encoded_length: usize,
            input: *const f32,
            input_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_matvec_owned(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            rows: usize,
            columns: usize,
            encoded: *const dmhip_buf,
            encoded_offset: usize,
            encoded_length: usize,
            input: *const f32,
            input_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_dequantize(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            encoded: *const dmhip_buf,
            encoded_offset: usize,
            encoded_length: usize,
            output: *mut f32,
            elements: usize,
        ) -> c_int;

        // stream-ordered device operators
        pub fn dmhip_matvec_device(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            rows: usize,
            columns: usize,
            weights: *const c_void,
            batch: usize,
            x: *const f32,
            y: *mut f32,
        ) -> c_int;
        pub fn dmhip_matvec_argmax_device(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            rows: usize,
            columns: usize,
            weights: *const c_void,
            x: *const f32,
            y: *mut f32,
            index_device: *mut u32,
        ) -> c_int;
        pub fn dmhip_argmax_result(ctx: *mut dmhip_ctx, index: *mut usize) -> c_int;
        pub fn dmhip_matvec_batch_device(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            rows: usize,
            columns: usize,
            count: usize,
            weights: *const *const c_void,
            x: *const f32,
            x_stride: usize,
            y: *mut f32,
            y_stride: usize,
        ) -> c_int;
        pub fn dmhip_rms_norm_device(
            ctx: *mut dmhip_ctx,
            batch: usize,
            count: usize,
            input: *const f32,
            weight: *const f32,
            epsilon: f32,
            output: *mut f32,
        ) -> c_int;
        pub fn dmhip_silu_mul_device(
            ctx: *mut dmhip_ctx,
            count: usize,
            gate: *const f32,
            up: *const f32,
            output: *mut f32,
        ) -> c_int;
        pub fn dmhip_softcap_device(
            ctx: *mut dmhip_ctx,
            count: usize,
            input: *const f32,
            cap: f32,
            output: *mut f32,
        ) -> c_int;
        pub fn dmhip_ffn_workspace_bytes(batch: usize, hidden: usize, ffn: usize) -> usize;
        pub fn dmhip_ffn_device(
            ctx: *mut dmhip_ctx,
            batch: usize,
            hidden: usize,
            ffn: usize,
            gate_type: u32,
            gate: *const c_void,
            up_type: u32,
            up: *const c_void,
            down_type: u32,
            down: *const c_void,
            epsilon: f32,
            h: *const f32,
            y: *mut f32,
            workspace: *mut c_void,
            workspace_len: usize,
        ) -> c_int;
        pub fn dmhip_ffn_noalloc_scratch_bytes() -> usize;
        pub fn dmhip_ffn_device_noalloc(
            ctx: *mut dmhip_ctx,
            batch: usize,
            hidden: usize,
            ffn: usize,
            gate_type: u32,
            gate: *const c_void,
            up_type: u32,
            up: *const c_void,
            down_type: u32,
            down: *const c_void,
            epsilon: f32,
            h: *const f32,
            y: *mut f32,
        ) -> c_int;
        pub fn dmhip_router_top_k_device(
            ctx: *mut dmhip_ctx,
            batch: usize,
            hidden: usize,
            experts: usize,
            k: usize,
            router_bf16: *const u16,
            x: *const f32,
            logits: *mut f32,
            ids: *mut u32,
            probabilities: *mut f32,
        ) -> c_int;
        pub fn dmhip_router_result(ctx: *mut dmhip_ctx) -> c_int;
        pub fn dmhip_gemm_workspace_bytes(m: usize, k: usize) -> usize;
        pub fn dmhip_gemm_device(
            ctx: *mut dmhip_ctx,
            ggml_type: u32,
            m: usize,
            n: usize,
            k: usize,
            a_bf16: *const u16,
            weights: *const c_void,
            c: *mut f32,
            workspace: *mut c_void,
            workspace_len: usize,
        ) -> c_int;

        // events and device copies
        pub fn dmhip_event_record(ctx: *mut dmhip_ctx, event: *mut *mut c_void) -> c_int;
        pub fn dmhip_event_elapsed_ms(start: *mut c_void, stop: *mut c_void, ms: *mut f32) -> c_int;
        pub fn dmhip_event_free(event: *mut c_void);
        pub fn dmhip_copy_device(ctx: *mut dmhip_ctx, dst: *mut c_void, src: *const c_void, n: usize) -> c_int;

        // routed-expert residency
        pub fn dmhip_expert_cache_new(
            ctx: *mut dmhip_ctx,
            source: *const c_void,
            source_len: usize,
            layouts: *const dmhip_expert_layer_layout,
            layer_count: usize,
            slots_per_layer: usize,
            out: *mut *mut dmhip_expert_cache,
        ) -> c_int;
        pub fn dmhip_expert_cache_new_file(
            ctx: *mut dmhip_ctx,
            fd: c_int,
            layouts: *const dmhip_expert_layer_layout,
            layer_count: usize,
            slots_per_layer: usize,
            out: *mut *mut dmhip_expert_cache,
        ) -> c_int;
        pub fn dmhip_expert_cache_free(cache: *mut dmhip_expert_cache);
        pub fn dmhip_expert_cache_stats_get(cache: *mut dmhip_expert_cache, stats: *mut dmhip_expert_cache_stats)
        -> c_int;
        pub fn dmhip_expert_cache_slots_per_layer(cache: *const dmhip_expert_cache) -> usize;
        pub fn dmhip_expert_acquire(
            cache: *mut dmhip_expert_cache,
            layer: usize,
            expert: usize,
            cancelled: *const c_int,
            slot: *mut usize,
            gate_up: *mut *const dmhip_buf,
            down: *mut *const dmhip_buf,
        ) -> c_int;
        pub fn dmhip_expert_release(cache: *mut dmhip_expert_cache, layer: usize, slot: usize) -> c_int;
        pub fn dmhip_moe_layer(
            ctx: *mut dmhip_ctx,
            cache: *mut dmhip_expert_cache,
            layer: usize,
            batch: usize,
            hidden: usize,
            width: usize,
            experts: usize,
            k: usize,
            router_bf16: *const u16,
            gate_up_type: u32,
            down_type: u32,
            x: *const f32,
            y: *mut f32,
            ids: *mut u32,
            probabilities: *mut f32,
        ) -> c_int;

        // GLM safetensors matrices
        pub fn dmhip_matvec_safetensor_mapped(
            ctx: *mut dmhip_ctx,
            safe_dtype: u32,
            rows: usize,
            columns: usize,
            mapping: *const dmhip_buf,
            encoded_offset: usize,
            encoded_length: usize,
            scale_mapping: *const dmhip_buf,
            scale_offset: usize,
            scale_length: usize,
            input: *const f32,
            input_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_matvec_safetensor(
            ctx: *mut dmhip_ctx,
            safe_dtype: u32,
            rows: usize,
            columns: usize,
            encoded: *const u8,
            encoded_len: usize,
            scales: *const f32,
            scales_len: usize,
            input: *const f32,
            input_len: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_matvec_safetensor_device(
            ctx: *mut dmhip_ctx,
            safe_dtype: u32,
            rows: usize,
            columns: usize,
            weights: *const c_void,
            weights_len: usize,
            scales: *const f32,
            scales_len: usize,
            x: *const f32,
            y: *mut f32,
        ) -> c_int;

        // decode attention over a KV ring
        pub fn dmhip_new_kv_layer(
            ctx: *mut dmhip_ctx,
            width: usize,
            max_context: usize,
            has_window: c_int,
            sliding_window: usize,
            out: *mut *mut dmhip_kv_layer,
        ) -> c_int;
        pub fn dmhip_kv_layer_free(layer: *mut dmhip_kv_layer);
        pub fn dmhip_kv_layer_position(layer: *const dmhip_kv_layer) -> usize;
        pub fn dmhip_kv_layer_capacity(layer: *const dmhip_kv_layer) -> usize;
        pub fn dmhip_kv_layer_allocated_bytes(layer: *const dmhip_kv_layer) -> usize;
        pub fn dmhip_kv_layer_clear(layer: *mut dmhip_kv_layer);
        pub fn dmhip_kv_layer_truncate(layer: *mut dmhip_kv_layer, position: usize);
        pub fn dmhip_kv_layer_width(layer: *const dmhip_kv_layer) -> usize;
        pub fn dmhip_kv_layer_keys(layer: *const dmhip_kv_layer) -> *mut c_void;
        pub fn dmhip_kv_layer_values(layer: *const dmhip_kv_layer) -> *mut c_void;
        pub fn dmhip_append_kv(
            ctx: *mut dmhip_ctx,
            layer: *mut dmhip_kv_layer,
            position: usize,
            key: *const f32,
            key_len: usize,
            value: *const f32,
            value_len: usize,
        ) -> c_int;
        pub fn dmhip_append_kv_device(
            ctx: *mut dmhip_ctx,
            layer: *mut dmhip_kv_layer,
            position: usize,
            key_device: *const f32,
            key_len: usize,
            value_device: *const f32,
            value_len: usize,
        ) -> c_int;
        pub fn dmhip_attention_cached(
            ctx: *mut dmhip_ctx,
            query: *const f32,
            query_len: usize,
            layer: *const dmhip_kv_layer,
            query_heads: usize,
            kv_heads: usize,
            head_dimension: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_attention_cached_device(
            ctx: *mut dmhip_ctx,
            query_device: *const f32,
            query_len: usize,
            layer: *const dmhip_kv_layer,
            query_heads: usize,
            kv_heads: usize,
            head_dimension: usize,
            output_device: *mut f32,
            output_len: usize,
        ) -> c_int;
        pub fn dmhip_attention_result(ctx: *mut dmhip_ctx) -> c_int;
        pub fn dmhip_attention(
            ctx: *mut dmhip_ctx,
            query: *const f32,
            query_len: usize,
            keys: *const f32,
            keys_len: usize,
            values: *const f32,
            values_len: usize,
            query_heads: usize,
            kv_heads: usize,
            head_dimension: usize,
            has_window: c_int,
            window: usize,
            output: *mut f32,
            output_len: usize,
        ) -> c_int;
    }
}

// ---------------------------------------------------------------------------
// Status -> MetalError / ExpertCacheError
// ---------------------------------------------------------------------------

/// The library's detail strings are string literals or entries of its
/// type-name table, alive as long as the library, which stays loaded for the
/// life of the process (it is linked, not opened at run time).
fn static_str(text: *const c_char) -> &'static str {
    if text.is_null() {
        return "";
    }
    // SAFETY: a NUL-terminated static string of the library (see above).
    let text: &'static CStr = unsafe { CStr::from_ptr(text) };
    text.to_str().unwrap_or("")
}

fn field(value: u64) -> usize {
    usize::try_from(value).unwrap_or(usize::MAX)
}

/// The calling thread's last failure: its payload and its message.
fn last_failure() -> (ffi::dmhip_error_detail, String) {
    let mut detail = ffi::dmhip_error_detail::empty();
    // SAFETY: `detail` is a valid out-pointer; both calls read thread-local state.
    unsafe { ffi::dmhip_last_error_detail(&mut detail) };
    let message = unsafe { CStr::from_ptr(ffi::dmhip_last_error()) }
        .to_string_lossy()
        .into_owned();
    (detail, message)
}

/// The `MetalError` variant a failed status mirrors, rebuilt with the fields
/// of the failure (src/metal.rs:3-126).
fn metal_error(code: c_int) -> MetalError {
    let (d, message) = last_failure();
    match code {
        ffi::DMHIP_ERR_NO_DEVICE => MetalError::NoDevice,
        ffi::DMHIP_ERR_BUFFER_ALLOCATION => MetalError::BufferAllocation { bytes: field(d.bytes) },
        ffi::DMHIP_ERR_VECTOR_LENGTH => MetalError::VectorLength {
            left: field(d.left),
            right: field(d.right),
            output: field(d.output),
        },
        ffi::DMHIP_ERR_VECTOR_TOO_LARGE => MetalError::VectorTooLarge,
        ffi::DMHIP_ERR_EMPTY_INPUT => MetalError::EmptyInput {
            operation: static_str(d.operation),
        },
        ffi::DMHIP_ERR_INVALID_VECTOR_LENGTH => MetalError::InvalidVectorLength {
            operation: static_str(d.operation),
            argument: static_str(d.argument),
            expected: field(d.expected),
            actual: field(d.actual),
        },
        ffi::DMHIP_ERR_INVALID_POSITIVE_PARAMETER => MetalError::InvalidPositiveParameter {
            operation: static_str(d.operation),
        },
        ffi::DMHIP_ERR_NON_FINITE => MetalError::NonFinite {
            operation: static_str(d.operation),
        },
        ffi::DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE => MetalError::UnsupportedTensorType(static_str(d.kind)),
        ffi::DMHIP_ERR_INVALID_ELEMENT_COUNT => MetalError::InvalidElementCount {
            kind: static_str(d.kind),
            elements: field(d.elements),
            block_elements: d.block_elements,
        },
        ffi::DMHIP_ERR_INVALID_BYTE_LENGTH => MetalError::InvalidByteLength {
            kind: static_str(d.kind),
            expected: field(d.expected),
            actual: field(d.actual),
        },
        ffi::DMHIP_ERR_OVERFLOW => MetalError::Overflow,
        ffi::DMHIP_ERR_INVALID_INPUT_LENGTH => MetalError::InvalidInputLength {
            expected: field(d.expected),
            actual: field(d.actual),
        },
        ffi::DMHIP_ERR_INVALID_OUTPUT_LENGTH => MetalError::InvalidOutputLength {
            expected: field(d.expected),
            actual: field(d.actual),
        },
        ffi::DMHIP_ERR_INVALID_TOP_K => MetalError::InvalidTopK {
            k: field(d.k),
            length: field(d.length),
        },
        ffi::DMHIP_ERR_MAPPED_RANGE => MetalError::MappedRange {
            offset: field(d.offset),
            end: field(d.end),
            length: field(d.length),
        },
        ffi::DMHIP_ERR_INVALID_ATTENTION_SHAPE => MetalError::InvalidAttentionShape(static_str(d.reason)),
        ffi::DMHIP_ERR_KV_POSITION => MetalError::KvPosition {
            expected: field(d.expected),
            actual: field(d.actual),
        },
        ffi::DMHIP_ERR_KV_WIDTH => MetalError::KvWidth {
            expected: field(d.expected),
            actual: field(d.actual),
        },
        ffi::DMHIP_ERR_KV_CONTEXT => MetalError::KvContext {
            position: field(d.position),
            limit: field(d.limit),
        },
        ffi::DMHIP_ERR_INVALID_ROPE_SHAPE => MetalError::InvalidRopeShape {
            length: field(d.length),
            heads: field(d.heads),
            head_dimension: field(d.head_dimension),
        },
        ffi::DMHIP_ERR_INVALID_ROPE_PAIRS => MetalError::InvalidRopePairs,
        // DMHIP_ERR_COMMAND (a HIP runtime error), DMHIP_ERR_INVALID_ARGUMENT
        // (a null handle: unreachable through this module) and an
        // expert-cache status reaching a context method: the message names
        // the failure.
        _ => MetalError::Command(message),
    }
}

fn check(code: c_int) -> Result<(), MetalError> {
    if code == ffi::DMHIP_OK { Ok(()) } else { Err(metal_error(code)) }
}

/// The `ExpertCacheError` variant a failed status mirrors
/// (src/expert.rs:13-42); context-level statuses become
/// `ExpertCacheError::Metal`.
fn cache_error(code: c_int) -> ExpertCacheError {
    let (d, message) = last_failure();
    match code {
        ffi::DMHIP_ERR_NO_SLOTS => ExpertCacheError::NoSlots,
        ffi::DMHIP_ERR_INVALID_LAYER => ExpertCacheError::InvalidLayer {
            layer: field(d.layer),
            count: field(d.count),
        },
        ffi::DMHIP_ERR_INVALID_EXPERT => ExpertCacheError::InvalidExpert {
            layer: field(d.layer),
            expert: field(d.expert),
            count: field(d.count),
        },
        ffi::DMHIP_ERR_ALL_SLOTS_PINNED => ExpertCacheError::AllSlotsPinned { layer: field(d.layer) },
        ffi::DMHIP_ERR_CANCELLED => ExpertCacheError::Cancelled,
        ffi::DMHIP_ERR_INVALID_LAYOUT => ExpertCacheError::InvalidLayout(message),
        // os_error 0 is the short read that read_exact_at reports as
        // UnexpectedEof (src/expert.rs:241-256)
        ffi::DMHIP_ERR_IO if d.os_error != 0 => ExpertCacheError::Io(io::Error::from_raw_os_error(d.os_error)),
        ffi::DMHIP_ERR_IO => {
            ExpertCacheError::Io(io::Error::new(io::ErrorKind::UnexpectedEof, "failed to fill whole buffer"))
        }
        _ => ExpertCacheError::Metal(metal_error(code)),
    }
}

fn cache_check(code: c_int) -> Result<(), ExpertCacheError> {
    if code == ffi::DMHIP_OK { Ok(()) } else { Err(cache_error(code)) }
}

/// ggml id of a tensor type (src/gguf.rs:295-318). The library reports
/// `UnsupportedTensorType` for the ids its kernels do not take.
fn ggml_id(kind: TensorType) -> u32 {
    match kind {
        TensorType::F32 => 0,
        TensorType::F16 => 1,
        TensorType::Q4_0 => 2,
        TensorType::Q4_1 => 3,
        TensorType::Q5_0 => 6,
        TensorType::Q5_1 => 7,
        TensorType::Q8_0 => 8,
        TensorType::Q8_1 => 9,
        TensorType::Q2K => 10,
        TensorType::Q3K => 11,
        TensorType::Q4K => 12,
        TensorType::Q5K => 13,
        TensorType::Q6K => 14,
        TensorType::Q8K => 15,
        TensorType::I8 => 24,
        TensorType::I16 => 25,
        TensorType::I32 => 26,
        TensorType::I64 => 27,
        TensorType::F64 => 28,
        TensorType::Bf16 => 30,
    }
}

/// SafeDtype id of the safetensors entry points (src/safetensors.rs:171-187).
fn safe_id(dtype: SafeDtype) -> u32 {
    match dtype {
        SafeDtype::Bool => ffi::DMHIP_SAFE_BOOL,
        SafeDtype::U8 => ffi::DMHIP_SAFE_U8,
        SafeDtype::I8 => ffi::DMHIP_SAFE_I8,
        SafeDtype::U16 => ffi::DMHIP_SAFE_U16,
        SafeDtype::I16 => ffi::DMHIP_SAFE_I16,
        SafeDtype::F16 => ffi::DMHIP_SAFE_F16,
        SafeDtype::Bf16 => ffi::DMHIP_SAFE_BF16,
        SafeDtype::U32 => ffi::DMHIP_SAFE_U32,
        SafeDtype::I32 => ffi::DMHIP_SAFE_I32,
        SafeDtype::F32 => ffi::DMHIP_SAFE_F32,
        SafeDtype::U64 => ffi::DMHIP_SAFE_U64,
        SafeDtype::I64 => ffi::DMHIP_SAFE_I64,
        SafeDtype::F64 => ffi::DMHIP_SAFE_F64,
        SafeDtype::F8E4M3 => ffi::DMHIP_SAFE_F8_E4M3,
        SafeDtype::F8E5M2 => ffi::DMHIP_SAFE_F8_E5M2,
    }
}

// ---------------------------------------------------------------------------
// Context and buffers
// ---------------------------------------------------------------------------

/// The library context, shared by the `MetalContext` and every buffer made
/// from it, and freed after the last of them. Neither `Send` nor `Sync`: the
/// library's context is used from one thread at a time, and DiskMule creates
/// and uses its context on the model-worker thread only
/// (src/runtime.rs:741-760).
struct Context {
    raw: NonNull<ffi::dmhip_ctx>,
}

impl Context {
    fn raw(&self) -> *mut ffi::dmhip_ctx {
        self.raw.as_ptr()
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        // SAFETY: the last owner of a live context; the library waits for the
        // context's streams before freeing it.
        unsafe { ffi::dmhip_context_free(self.raw.as_ptr()) }
    }
}

/// MetalContext (src/metal.rs:180-205), backed by one HIP device and its
/// compute and upload streams. Every method validates its arguments in the
/// reference's order, runs on the GPU and returns after the work finished,
/// as src/metal.rs:1595-1596 does.
pub struct MetalContext {
    context: Rc<Context>,
}

/// MetalMappedBuffer (src/metal.rs:207-211): the GGUF mapping, uploaded to HBM
/// once by `map_read_only` with its byte offsets kept. The `Arc<Mmap>` is
/// held as the Metal buffer holds it.
pub struct MetalMappedBuffer {
    context: Rc<Context>,
    raw: NonNull<ffi::dmhip_buf>,
    mapping: Arc<Mmap>,
}

/// MetalOwnedBuffer (src/metal.rs:213-243): device memory owned by the
/// buffer, or an expert slot lent by `ExpertCache::with_expert` (`owned`
/// false: the cache frees it). HBM is not host-addressable, so `as_bytes`
/// returns a copy and writes go through `write_bytes`.
pub struct MetalOwnedBuffer {
    context: Rc<Context>,
    raw: NonNull<ffi::dmhip_buf>,
    owned: bool,
}

/// MetalKvLayer (src/metal.rs:245-278): the key and value rings of one
/// layer in HBM, `capacity` slots of `width` floats each, with the position
/// kept by the library.
pub struct MetalKvLayer {
    context: Rc<Context>,
    raw: NonNull<ffi::dmhip_kv_layer>,
}

impl fmt::Debug for MetalContext {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("MetalContext").field("device", &self.device_name()).finish()
    }
}

impl fmt::Debug for MetalMappedBuffer {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("MetalMappedBuffer").field("length", &self.len()).finish()
    }
}

impl fmt::Debug for MetalOwnedBuffer {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("MetalOwnedBuffer")
            .field("length", &self.len())
            .field("owned", &self.owned)
            .finish()
    }
}

impl fmt::Debug for MetalKvLayer {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("MetalKvLayer")
            .field("position", &self.position())
            .field("capacity", &self.capacity())
            .finish()
    }
}

impl Drop for MetalKvLayer {
    fn drop(&mut self) {
        // SAFETY: the layer is live and its context outlives it (Rc); the
        // library waits for the context's stream before freeing the rings.
        unsafe { ffi::dmhip_kv_layer_free(self.raw.as_ptr()) }
    }
}

impl Drop for MetalMappedBuffer {
    fn drop(&mut self) {
        // SAFETY: the buffer is live and its context outlives it (Rc).
        unsafe { ffi::dmhip_buffer_free(self.raw.as_ptr()) }
    }
}

impl Drop for MetalOwnedBuffer {
    fn drop(&mut self) {
        if self.owned {
            // SAFETY: as for MetalMappedBuffer.
            unsafe { ffi::dmhip_buffer_free(self.raw.as_ptr()) }
        }
    }
}

impl MetalMappedBuffer {
    pub fn len(&self) -> usize {
        self.mapping.len()
    }

    pub fn is_empty(&self) -> bool {
        self.mapping.is_empty()
    }
}

impl MetalOwnedBuffer {
    pub fn len(&self) -> usize {
        // SAFETY: the buffer is live.
        unsafe { ffi::dmhip_buffer_len(self.raw.as_ptr()) }
    }

    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }

    /// The buffer's bytes, copied from HBM after the work enqueued on the
    /// context so far (src/metal.rs:228-234 returns the shared memory itself).
    pub fn as_bytes(&self) -> Vec<u8> {
        let mut bytes = vec![0_u8; self.len()];
        // SAFETY: `bytes` holds len() bytes; the buffer and its context are live.
        let code = unsafe {
            ffi::dmhip_buffer_read(
                self.context.raw(),
                self.raw.as_ptr(),
                0,
                bytes.as_mut_ptr().cast(),
                bytes.len(),
            )
        };
        // a failed copy is a HIP runtime error on a live buffer: a broken device
        check(code).expect("reading a device buffer failed");
        bytes
    }

    /// Writes `bytes` at `offset` (the role of src/metal.rs:236-243's
    /// as_mut_bytes). A range past the end is MappedRange.
    pub fn write_bytes(&mut self, offset: usize, bytes: &[u8]) -> Result<(), MetalError> {
        // SAFETY: the library checks the range against the buffer's length.
        check(unsafe {
            ffi::dmhip_buffer_write(
                self.context.raw(),
                self.raw.as_ptr(),
                offset,
                bytes.as_ptr().cast(),
                bytes.len(),
            )
        })
    }
}

impl MetalKvLayer {
    pub fn position(&self) -> usize {
        // SAFETY: the layer is live (all five are host-side bookkeeping).
        unsafe { ffi::dmhip_kv_layer_position(self.raw.as_ptr()) }
    }

    pub fn capacity(&self) -> usize {
        unsafe { ffi::dmhip_kv_layer_capacity(self.raw.as_ptr()) }
    }

    pub fn allocated_bytes(&self) -> usize {
        unsafe { ffi::dmhip_kv_layer_allocated_bytes(self.raw.as_ptr()) }
    }

    pub fn clear(&mut self) {
        unsafe { ffi::dmhip_kv_layer_clear(self.raw.as_ptr()) }
    }

    pub fn truncate(&mut self, position: usize) {
        unsafe { ffi::dmhip_kv_layer_truncate(self.raw.as_ptr(), position) }
    }
}
impl MetalContext {
    /// MetalContext::new (src/metal.rs:291-346) on HIP device 0 (the first
    /// device HIP_VISIBLE_DEVICES leaves visible). No device: NoDevice.
    pub fn new() -> Result<Self, MetalError> {
        let mut raw = ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer.
        check(unsafe { ffi::dmhip_context_new(0, &mut raw) })?;
        let raw = NonNull::new(raw).ok_or(MetalError::NoDevice)?;
        Ok(Self {
            context: Rc::new(Context { raw }),
        })
    }

    fn raw(&self) -> *mut ffi::dmhip_ctx {
        self.context.raw()
    }

    /// MetalContext::device_name (src/metal.rs:348-350).
    pub fn device_name(&self) -> String {
        let mut name = [0 as c_char; 256];
        // SAFETY: the library writes a NUL-terminated name of at most 256 bytes.
        let code = unsafe { ffi::dmhip_device_name(self.raw(), name.as_mut_ptr(), name.len()) };
        if code != ffi::DMHIP_OK {
            return String::from("HIP device");
        }
        unsafe { CStr::from_ptr(name.as_ptr()) }.to_string_lossy().into_owned()
    }

    /// MetalContext::map_read_only (src/metal.rs:352-392). A discrete GPU
    /// cannot wrap the host mapping, so the whole mapping is uploaded to HBM
    /// once; offsets into it stay file offsets. An empty mapping is
    /// BufferAllocation { bytes: 0 }, as in the reference.
    pub fn map_read_only(&self, mapping: Arc<Mmap>) -> Result<MetalMappedBuffer, MetalError> {
        let mut raw = ptr::null_mut();
        // SAFETY: the mapping is readable for its length during the call.
        check(unsafe { ffi::dmhip_map_read_only(self.raw(), mapping.as_ptr().cast(), mapping.len(), &mut raw) })?;
        let raw = NonNull::new(raw).ok_or(MetalError::BufferAllocation { bytes: mapping.len() })?;
        Ok(MetalMappedBuffer {
            context: Rc::clone(&self.context),
            raw,
            mapping,
        })
    }

    /// MetalContext::new_owned_buffer (src/metal.rs:394-402): zero-filled.
    pub fn new_owned_buffer(&self, length: usize) -> Result<MetalOwnedBuffer, MetalError> {
        let mut raw = ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer.
        check(unsafe { ffi::dmhip_new_owned_buffer(self.raw(), length, &mut raw) })?;
        let raw = NonNull::new(raw).ok_or(MetalError::BufferAllocation { bytes: length })?;
        Ok(MetalOwnedBuffer {
            context: Rc::clone(&self.context),
            raw,
            owned: true,
        })
    }

    /// MetalContext::rms_norm (src/metal.rs:435-476).
    pub fn rms_norm(
        &self,
        input: &[f32],
        weight: Option<&[f32]>,
        epsilon: f32,
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        let (weight_ptr, weight_len) = weight.map_or((ptr::null(), 0), |w| (w.as_ptr(), w.len()));
        // SAFETY: every pointer comes with its slice length.
        check(unsafe {
            ffi::dmhip_rms_norm(
                self.raw(),
                input.as_ptr(),
                input.len(),
                weight_ptr,
                weight_len,
                epsilon,
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::silu_mul (src/metal.rs:554-576).
    pub fn silu_mul(&self, gate: &[f32], up: &[f32], output: &mut [f32]) -> Result<(), MetalError> {
        // SAFETY: as above.
        check(unsafe {
            ffi::dmhip_silu_mul(
                self.raw(),
                gate.as_ptr(),
                gate.len(),
                up.as_ptr(),
                up.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::softcap (src/metal.rs:600-622).
    pub fn softcap(&self, input: &[f32], cap: f32, output: &mut [f32]) -> Result<(), MetalError> {
        // SAFETY: as above.
        check(unsafe {
            ffi::dmhip_softcap(
                self.raw(),
                input.as_ptr(),
                input.len(),
                cap,
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::argmax (src/metal.rs:624-644).
    pub fn argmax(&self, input: &[f32]) -> Result<usize, MetalError> {
        let mut index = 0_usize;
        // SAFETY: as above.
        check(unsafe { ffi::dmhip_argmax(self.raw(), input.as_ptr(), input.len(), &mut index) })?;
        Ok(index)
    }

    /// MetalContext::top_k_softmax (src/metal.rs:1392-1434). The id and
    /// probability arrays are sized by the library's own check (InvalidTopK
    /// for k outside 1..=len) before any write.
    pub fn top_k_softmax(&self, logits: &[f32], k: usize) -> Result<Vec<(usize, f32)>, MetalError> {
        let size = if k >= 1 && k <= logits.len() { k } else { 0 };
        let mut indices = vec![0_usize; size];
        let mut probabilities = vec![0_f32; size];
        // SAFETY: the library writes k entries only after k passed its check,
        // and then `size == k`.
        check(unsafe {
            ffi::dmhip_top_k_softmax(
                self.raw(),
                logits.as_ptr(),
                logits.len(),
                k,
                indices.as_mut_ptr(),
                probabilities.as_mut_ptr(),
            )
        })?;
        Ok(indices.into_iter().zip(probabilities).collect())
    }

    /// MetalContext::matvec (src/metal.rs:648-683).
    pub fn matvec(
        &self,
        kind: TensorType,
        rows: usize,
        columns: usize,
        encoded: &[u8],
        input: &[f32],
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        // SAFETY: as above.
        check(unsafe {
            ffi::dmhip_matvec(
                self.raw(),
                ggml_id(kind),
                rows,
                columns,
                encoded.as_ptr(),
                encoded.len(),
                input.as_ptr(),
                input.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::matvec_mapped (src/metal.rs:687-734): the check order of
    /// prepare_matvec (src/metal.rs:1513-1560), then MappedRange.
    pub fn matvec_mapped(
        &self,
        kind: TensorType,
        rows: usize,
        columns: usize,
        mapping: &MetalMappedBuffer,
        encoded_offset: usize,
        encoded_length: usize,
        input: &[f32],
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        // SAFETY: as above; the library bounds the range by the mapping.
        check(unsafe {
            ffi::dmhip_matvec_mapped(
                self.raw(),
                ggml_id(kind),
                rows,
                columns,
                mapping.raw.as_ptr(),
                encoded_offset,
                encoded_length,
                input.as_ptr(),
                input.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::matvec_owned (src/metal.rs:1148-1194), including an
    /// expert slot lent by `ExpertCache::with_expert`.
    pub fn matvec_owned(
        &self,
        kind: TensorType,
        rows: usize,
        columns: usize,
        encoded: &MetalOwnedBuffer,
        encoded_offset: usize,
        encoded_length: usize,
        input: &[f32],
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        // SAFETY: as above.
        check(unsafe {
            ffi::dmhip_matvec_owned(
                self.raw(),
                ggml_id(kind),
                rows,
                columns,
                encoded.raw.as_ptr(),
                encoded_offset,
                encoded_length,
                input.as_ptr(),
                input.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::add (src/metal.rs:404-432).
    pub fn add(&self, left: &[f32], right: &[f32], output: &mut [f32]) -> Result<(), MetalError> {
        // SAFETY: the slices are valid for their lengths for the call; the
        // library checks the lengths before it touches them.
        check(unsafe {
            ffi::dmhip_add(
                self.raw(),
                left.as_ptr(),
                left.len(),
                right.as_ptr(),
                right.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::rope_neox_in_place (src/metal.rs:478-528).
    pub fn rope_neox_in_place(
        &self,
        values: &mut [f32],
        heads: usize,
        head_dimension: usize,
        rotated_pairs: usize,
        position: usize,
        theta: f32,
    ) -> Result<(), MetalError> {
        // SAFETY: as above.
        check(unsafe {
            ffi::dmhip_rope_neox_in_place(
                self.raw(),
                values.as_mut_ptr(),
                values.len(),
                heads,
                head_dimension,
                rotated_pairs,
                position,
                theta,
            )
        })
    }

    /// MetalContext::gelu_mul (src/metal.rs:530-552).
    pub fn gelu_mul(&self, gate: &[f32], up: &[f32], output: &mut [f32]) -> Result<(), MetalError> {
        // SAFETY: as above.
        check(unsafe {
            ffi::dmhip_gelu_mul(
                self.raw(),
                gate.as_ptr(),
                gate.len(),
                up.as_ptr(),
                up.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    /// MetalContext::softmax (src/metal.rs:578-598).
    pub fn softmax(&self, input: &[f32], output: &mut [f32]) -> Result<(), MetalError> {
        // SAFETY: as above.
        check(unsafe {
            ffi::dmhip_softmax(self.raw(), input.as_ptr(), input.len(), output.as_mut_ptr(), output.len())
        })
    }

    pub fn matvec_safetensor_mapped(
        &self,
        dtype: SafeDtype,
        rows: usize,
        columns: usize,
        mapping: &MetalMappedBuffer,
        encoded_offset: usize,
        encoded_length: usize,
        scale: Option<(&MetalMappedBuffer, usize, usize)>,
        input: &[f32],
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        let (scale_raw, scale_offset, scale_length) = match scale {
            Some((buffer, offset, length)) => (buffer.raw.as_ptr().cast_const(), offset, length),
            None => (ptr::null(), 0, 0),
        };
        // SAFETY: the buffers belong to live contexts; the library checks
        // both ranges against their mappings and the slices' lengths.
        check(unsafe {
            ffi::dmhip_matvec_safetensor_mapped(
                self.context.raw(),
                safe_id(dtype),
                rows,
                columns,
                mapping.raw.as_ptr(),
                encoded_offset,
                encoded_length,
                scale_raw,
                scale_offset,
                scale_length,
                input.as_ptr(),
                input.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    pub fn matvec_safetensor(
        &self,
        dtype: SafeDtype,
        rows: usize,
        columns: usize,
        encoded: &[u8],
        scales: Option<&[f32]>,
        input: &[f32],
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        // None is a null pointer; Some(&[]) keeps its non-null dangling one
        let (scales_ptr, scales_len) = scales.map_or((ptr::null(), 0), |s| (s.as_ptr(), s.len()));
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            ffi::dmhip_matvec_safetensor(
                self.context.raw(),
                safe_id(dtype),
                rows,
                columns,
                encoded.as_ptr(),
                encoded.len(),
                scales_ptr,
                scales_len,
                input.as_ptr(),
                input.len(),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    pub fn new_kv_layer(
        &self,
        width: usize,
        max_context: usize,
        sliding_window: Option<usize>,
    ) -> Result<MetalKvLayer, MetalError> {
        let mut raw = ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer; the context is live.
        check(unsafe {
            ffi::dmhip_new_kv_layer(
                self.context.raw(),
                width,
                max_context,
                c_int::from(sliding_window.is_some()),
                sliding_window.unwrap_or(0),
                &mut raw,
            )
        })?;
        let raw = NonNull::new(raw).ok_or(MetalError::BufferAllocation { bytes: 0 })?;
        Ok(MetalKvLayer {
            context: Rc::clone(&self.context),
            raw,
        })
    }

    pub fn append_kv(
        &self,
        layer: &mut MetalKvLayer,
        position: usize,
        key: &[f32],
        value: &[f32],
    ) -> Result<(), MetalError> {
        // SAFETY: the slices are valid for their lengths; the library checks
        // them against the layer's width before copying.
        check(unsafe {
            ffi::dmhip_append_kv(
                self.context.raw(),
                layer.raw.as_ptr(),
                position,
                key.as_ptr(),
                key.len(),
                value.as_ptr(),
                value.len(),
            )
        })
    }

    pub fn attention_cached(
        &self,
        query: &[f32],
        cache: &MetalKvLayer,
        query_heads: usize,
        kv_heads: usize,
        head_dimension: usize,
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        // SAFETY: as for append_kv; the layer belongs to a live context.
        check(unsafe {
            ffi::dmhip_attention_cached(
                self.context.raw(),
                query.as_ptr(),
                query.len(),
                cache.raw.as_ptr(),
                query_heads,
                kv_heads,
                head_dimension,
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }

    pub fn attention(
        &self,
        query: &[f32],
        keys: &[f32],
        values: &[f32],
        query_heads: usize,
        kv_heads: usize,
        head_dimension: usize,
        window: Option<usize>,
        output: &mut [f32],
    ) -> Result<(), MetalError> {
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            ffi::dmhip_attention(
                self.context.raw(),
                query.as_ptr(),
                query.len(),
                keys.as_ptr(),
                keys.len(),
                values.as_ptr(),
                values.len(),
                query_heads,
                kv_heads,
                head_dimension,
                c_int::from(window.is_some()),
                window.unwrap_or(0),
                output.as_mut_ptr(),
                output.len(),
            )
        })
    }
}

// ---------------------------------------------------------------------------
// Routed-expert residency
// ---------------------------------------------------------------------------

/// ExpertCache (src/expert.rs:64-164) over the GGUF file: per layer
/// `slots_per_layer` HBM slots, the reference's LRU victim rule and counters,
/// and misses read with two parallel positional reads into pinned staging
/// and copied into the slot on an upload stream that the compute stream
/// waits for.
pub struct ExpertCache {
    context: Rc<Context>,
    raw: NonNull<ffi::dmhip_expert_cache>,
    // the library reads the descriptor on every miss
    _file: Arc<File>,
}

impl fmt::Debug for ExpertCache {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("ExpertCache")
            .field("slots_per_layer", &self.slots_per_layer())
            .field("stats", &self.stats())
            .finish()
    }
}

impl Drop for ExpertCache {
    fn drop(&mut self) {
        // SAFETY: the cache is live; the library waits for its uploads and
        // for the work released from its slots before freeing them.
        unsafe { ffi::dmhip_expert_cache_free(self.raw.as_ptr()) }
    }
}

/// A slot pinned by `dmhip_expert_acquire`, released when dropped (also on
/// an early return or a panic in the closure).
struct SlotPin {
    cache: NonNull<ffi::dmhip_expert_cache>,
    layer: usize,
    slot: usize,
}

impl Drop for SlotPin {
    fn drop(&mut self) {
        // SAFETY: the slot was pinned by this pin's acquire; release records
        // the work enqueued so far as the slot's last use.
        let code = unsafe { ffi::dmhip_expert_release(self.cache.as_ptr(), self.layer, self.slot) };
        debug_assert_eq!(code, ffi::DMHIP_OK);
    }
}

impl ExpertCache {
    /// ExpertCache::new (src/expert.rs:88-128): NoSlots for zero slots,
    /// InvalidLayout for ranges that overflow, BufferAllocation (as
    /// ExpertCacheError::Metal) when HBM runs out.
    pub fn new(
        metal: &MetalContext,
        file: Arc<File>,
        layouts: &[ExpertLayerLayout],
        slots_per_layer: usize,
    ) -> Result<Self, ExpertCacheError> {
        let raw_layouts: Vec<ffi::dmhip_expert_layer_layout> = layouts
            .iter()
            .map(|layout| ffi::dmhip_expert_layer_layout {
                expert_count: layout.expert_count,
                gate_up_offset: layout.gate_up_offset,
                gate_up_bytes: layout.gate_up_bytes,
                down_offset: layout.down_offset,
                down_bytes: layout.down_bytes,
            })
            .collect();
        let mut raw = ptr::null_mut();
        // SAFETY: the layouts are valid for the call; the descriptor stays
        // open while the cache holds `file`.
        cache_check(unsafe {
            ffi::dmhip_expert_cache_new_file(
                metal.raw(),
                file.as_raw_fd(),
                raw_layouts.as_ptr(),
                raw_layouts.len(),
                slots_per_layer,
                &mut raw,
            )
        })?;
        let raw = NonNull::new(raw).ok_or(ExpertCacheError::NoSlots)?;
        Ok(Self {
            context: Rc::clone(&metal.context),
            raw,
            _file: file,
        })
    }

    /// ExpertCache::stats (src/expert.rs:130-132). io_wait is the host's wall
    /// time in the positional reads, as src/expert.rs:220 measures it.
    pub fn stats(&self) -> ExpertCacheStats {
        let mut stats = ffi::dmhip_expert_cache_stats::default();
        // SAFETY: the cache is live; the call fails only for a null handle.
        unsafe { ffi::dmhip_expert_cache_stats_get(self.raw.as_ptr(), &mut stats) };
        ExpertCacheStats {
            hits: stats.hits,
            misses: stats.misses,
            evictions: stats.evictions,
            reads: stats.reads,
            bytes_read: stats.bytes_read,
            io_wait: Duration::from_nanos(stats.io_wait_ns),
            resident_bytes: stats.resident_bytes,
        }
    }

    pub fn slots_per_layer(&self) -> usize {
        // SAFETY: the cache is live.
        unsafe { ffi::dmhip_expert_cache_slots_per_layer(self.raw.as_ptr()) }
    }

    /// ExpertCache::with_expert (src/expert.rs:138-164): `cancelled` is
    /// checked before and after the acquire; the slot stays pinned while
    /// `use_expert` runs and is released after it (the release records the
    /// work the closure enqueued, so a later upload into the slot waits for
    /// it). The closure receives the slot's gate_up and down bytes as
    /// `&MetalOwnedBuffer`, which `matvec_owned` takes.
    pub fn with_expert<T, E, F, C>(&mut self, layer: usize, expert: usize, cancelled: C, use_expert: F) -> Result<T, E>
    where
        E: From<ExpertCacheError>,
        F: FnOnce(&MetalOwnedBuffer, &MetalOwnedBuffer) -> Result<T, E>,
        C: Fn() -> bool,
    {
        if cancelled() {
            return Err(ExpertCacheError::Cancelled.into());
        }
        let mut slot = 0_usize;
        let mut gate_up = ptr::null();
        let mut down = ptr::null();
        // SAFETY: valid out-pointers; no C-side cancel flag (checked here).
        let code = unsafe {
            ffi::dmhip_expert_acquire(self.raw.as_ptr(), layer, expert, ptr::null(), &mut slot, &mut gate_up, &mut down)
        };
        if code != ffi::DMHIP_OK {
            return Err(cache_error(code).into());
        }
        let pin = SlotPin {
            cache: self.raw,
            layer,
            slot,
        };
        if cancelled() {
            return Err(ExpertCacheError::Cancelled.into());
        }
        let lend = |raw: *const ffi::dmhip_buf| MetalOwnedBuffer {
            context: Rc::clone(&self.context),
            raw: NonNull::new(raw.cast_mut()).expect("acquire returns both slot buffers"),
            owned: false,
        };
        let (gate_up, down) = (lend(gate_up), lend(down));
        let result = use_expert(&gate_up, &down);
        drop(pin);
        result
    }
}

#[cfg(test)]
mod tests {
    //! The reference's own tests of this surface (src/expert.rs:258-325,
    //! src/metal.rs:2040-2142), which run unchanged on a GPU host.
    use std::io::Write;

    use super::*;

    #[test]
    fn bounded_cache_tracks_hits_misses_evictions_and_cancellation() {
        let metal = MetalContext::new().unwrap();
        let mut file = tempfile::tempfile().unwrap();
        file.write_all(&[1, 2, 3, 4, 5, 6, 7, 8, 11, 12, 13, 14, 15, 16, 17, 18]).unwrap();
        file.flush().unwrap();
        let layout = ExpertLayerLayout {
            expert_count: 2,
            gate_up_offset: 0,
            gate_up_bytes: 4,
            down_offset: 8,
            down_bytes: 4,
        };
        let mut cache = ExpertCache::new(&metal, Arc::new(file), &[layout], 1).unwrap();
        assert_eq!(cache.slots_per_layer(), 1);
        for _ in 0..2 {
            cache
                .with_expert::<_, ExpertCacheError, _, _>(0, 0, || false, |gate, down| {
                    assert_eq!(gate.as_bytes(), [1, 2, 3, 4]);
                    assert_eq!(down.as_bytes(), [11, 12, 13, 14]);
                    Ok(())
                })
                .unwrap();
        }
        cache
            .with_expert::<_, ExpertCacheError, _, _>(0, 1, || false, |gate, down| {
                assert_eq!(gate.as_bytes(), [5, 6, 7, 8]);
                assert_eq!(down.as_bytes(), [15, 16, 17, 18]);
                Ok(())
            })
            .unwrap();
        let stats = cache.stats();
        assert_eq!((stats.hits, stats.misses, stats.evictions), (1, 2, 1));
        assert_eq!((stats.reads, stats.bytes_read, stats.resident_bytes), (4, 16, 8));
        assert!(stats.io_wait > Duration::ZERO);
        assert!(matches!(
            cache.with_expert::<_, ExpertCacheError, _, _>(0, 0, || true, |_, _| Ok(())),
            Err(ExpertCacheError::Cancelled)
        ));
    }

    #[test]
    fn validation_errors_carry_the_reference_payloads() {
        let metal = MetalContext::new().unwrap();
        let mut output = [0.0_f32; 2];
        assert_eq!(
            metal.matvec(TensorType::Q8_0, 2, 32, &[0; 68], &[0.0; 31], &mut output),
            Err(MetalError::InvalidInputLength { expected: 32, actual: 31 })
        );
        assert_eq!(
            metal.matvec(TensorType::Q8_0, 2, 32, &[0; 67], &[0.0; 32], &mut output),
            Err(MetalError::InvalidByteLength { kind: "Q8_0", expected: 68, actual: 67 })
        );
        assert_eq!(
            metal.top_k_softmax(&[1.0, 2.0], 3),
            Err(MetalError::InvalidTopK { k: 3, length: 2 })
        );
        assert_eq!(
            metal.softcap(&[], 30.0, &mut []),
            Err(MetalError::EmptyInput { operation: "logit softcap" })
        );
    }
}
