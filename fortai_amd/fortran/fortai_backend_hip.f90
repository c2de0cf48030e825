! fortai_backend_hip.f90 -- Fortran (iso_c_binding) face of libfortai_hip.so.
!
! The public surface is the reference's device binding
! (src/backend/cuda/fortai_backend_cuda.f90:10-65): the same four derived types
! with the same type-bound procedures and the same free procedures, with the
! same argument lists and status behaviour, but named hip_* and bound to the
! fortai_hip_* C entry points (include/fortai_hip_backend.h).  Two additions:
! the C library's detailed error text reaches status_t%message, and the fused
! whole-token decoder (hip_qwen35_decoder_t) plus fp16 weights
! (hip_f16_weights_t) are exposed for callers that want one graph per token.
!
! Status contract (as the reference binding): invalid handles or sizes give
! FORTAI_INVALID before any C call; a non-zero C return gives
! FORTAI_UNSUPPORTED.  Destroying a null handle is a no-op.
!
! fortai_backend_cuda_on_hip.f90 re-exports this module under the reference's
! cuda_* names so the reference model compiles against it unchanged.
module fortai_backend_hip
    use, intrinsic :: iso_c_binding, only: c_associated, c_char, c_f_pointer, c_float, c_int, &
        c_int8_t, c_int16_t, c_int64_t, c_loc, c_null_char, c_null_ptr, c_ptr, c_size_t
    use fortai_status, only: FORTAI_INVALID, FORTAI_UNSUPPORTED, status_t
    implicit none
    private

    integer(c_int), parameter, public :: FORTAI_HIP_OK = 0_c_int

    type, public :: hip_q8_context_t
        type(c_ptr) :: handle = c_null_ptr
    contains
        procedure :: create => context_create
        procedure :: destroy => context_destroy
        procedure :: set_position => context_set_position
        procedure :: capture_begin => context_capture_begin
        procedure :: capture_end => context_capture_end
        procedure :: graph_launch => context_graph_launch
        procedure :: synchronize => context_synchronize
        procedure :: allocate_buffer => context_allocate_buffer
        procedure :: free_buffer => context_free_buffer
        procedure :: upload => context_upload
        procedure :: upload_real => context_upload_real
        procedure :: download => context_download
        procedure :: download_real => context_download_real
        procedure :: last_error => context_last_error
    end type hip_q8_context_t

    type, public :: hip_q8_weights_t
        type(c_ptr) :: handle = c_null_ptr
    contains
        procedure :: upload => q8_weights_upload
        procedure :: destroy => q8_weights_destroy
        procedure :: pack => q8_weights_pack
        procedure :: upload_packed => q8_weights_upload_packed
    end type hip_q8_weights_t

    type, public :: hip_f16_weights_t
        type(c_ptr) :: handle = c_null_ptr
    contains
        procedure :: upload => f16_weights_upload
        procedure :: destroy => f16_weights_destroy
    end type hip_f16_weights_t

    type, public :: hip_qwen35_recurrent_t
        type(c_ptr) :: handle = c_null_ptr
        type(c_ptr) :: context = c_null_ptr
    contains
        procedure :: create => recurrent_create
        procedure :: destroy => recurrent_destroy
        procedure :: reset => recurrent_reset
        procedure :: run => recurrent_run
        procedure :: run_device => recurrent_run_device
    end type hip_qwen35_recurrent_t

    type, public :: hip_qwen35_attention_t
        type(c_ptr) :: handle = c_null_ptr
        type(c_ptr) :: context = c_null_ptr
    contains
        procedure :: create => attention_create
        procedure :: destroy => attention_destroy
        procedure :: reset => attention_reset
        procedure :: run_device => attention_run_device
    end type hip_qwen35_attention_t

    type, public :: hip_qwen35_decoder_t
        type(c_ptr) :: handle = c_null_ptr
        type(c_ptr) :: context = c_null_ptr
    contains
        procedure :: create => decoder_create
        procedure :: destroy => decoder_destroy
        procedure :: reset => decoder_reset
        procedure :: forward => decoder_forward
        procedure :: generate => decoder_generate
        procedure :: plan => decoder_plan
    end type hip_qwen35_decoder_t

    ! Independent sequences (up to 8) over one set of layers and weights, with
    ! a prompt prefill on the i8 matrix cores (fortai_hip_qwen35_batch_*).
    type, public :: hip_qwen35_batch_t
        type(c_ptr) :: handle = c_null_ptr
        type(c_ptr) :: context = c_null_ptr
        integer :: batch = 0
    contains
        procedure :: create => batch_create
        procedure :: destroy => batch_destroy
        procedure :: reset => batch_reset
        procedure :: prefill => batch_prefill
        procedure :: generate => batch_generate
        procedure :: plan => batch_plan
    end type hip_qwen35_batch_t

    public :: hip_q8_pack_bytes
    public :: hip_q8_matvec_resident, hip_q8_matvec_device_f32, hip_qwen35_embedding_device
    public :: hip_qwen35_copy_device, hip_qwen35_add_device, hip_qwen35_rms_norm_device
    public :: hip_q8_matvec_host, hip_q8_matvec_host_pair, hip_q8_matvec_host_triplet
    public :: hip_q8_matvec_host_triplet_contiguous, hip_q8_ffn_host, hip_q8_ffn_device

    ! ---- C entry points (every pointer by value, sizes by value) -------------
    interface
        integer(c_int) function fh_context_create(device, context) &
                bind(C, name='fortai_hip_q8_context_create')
            import :: c_int, c_ptr
            integer(c_int), value :: device
            type(c_ptr), intent(out) :: context
        end function
        integer(c_int) function fh_context_call(context) bind(C, name='fortai_hip_q8_context_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: context
        end function
        integer(c_int) function fh_capture_begin(context) bind(C, name='fortai_hip_q8_context_capture_begin')
            import :: c_int, c_ptr
            type(c_ptr), value :: context
        end function
        integer(c_int) function fh_capture_end(context) bind(C, name='fortai_hip_q8_context_capture_end')
            import :: c_int, c_ptr
            type(c_ptr), value :: context
        end function
        integer(c_int) function fh_graph_launch(context) bind(C, name='fortai_hip_q8_context_graph_launch')
            import :: c_int, c_ptr
            type(c_ptr), value :: context
        end function
        integer(c_int) function fh_synchronize(context) bind(C, name='fortai_hip_q8_context_synchronize')
            import :: c_int, c_ptr
            type(c_ptr), value :: context
        end function
        integer(c_int) function fh_set_position(context, position) &
                bind(C, name='fortai_hip_q8_context_set_position')
            import :: c_int, c_ptr
            type(c_ptr), value :: context
            integer(c_int), value :: position
        end function
        type(c_ptr) function fh_last_error(context) bind(C, name='fortai_hip_q8_last_error')
            import :: c_ptr
            type(c_ptr), value :: context
        end function
        integer(c_int) function fh_weights_upload(context, host, bytes, rows, width, weights) &
                bind(C, name='fortai_hip_q8_weights_upload')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, host
            integer(c_size_t), value :: bytes
            integer(c_int), value :: rows, width
            type(c_ptr), intent(out) :: weights
        end function
        integer(c_int) function fh_weights_destroy(weights) bind(C, name='fortai_hip_q8_weights_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: weights
        end function
        integer(c_size_t) function fh_pack_bytes(rows, width) bind(C, name='fortai_hip_q8_pack_bytes')
            import :: c_int, c_size_t
            integer(c_int), value :: rows, width
        end function
        integer(c_int) function fh_weights_pack(weights, host, bytes) bind(C, name='fortai_hip_q8_weights_pack')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: weights, host
            integer(c_size_t), value :: bytes
        end function
        integer(c_int) function fh_weights_upload_packed(context, host, bytes, rows, width, weights) &
                bind(C, name='fortai_hip_q8_weights_upload_packed')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, host
            integer(c_size_t), value :: bytes
            integer(c_int), value :: rows, width
            type(c_ptr), intent(out) :: weights
        end function
        integer(c_int) function fh_f16_upload(context, host, bytes, rows, width, weights) &
                bind(C, name='fortai_hip_f16_weights_upload')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, host
            integer(c_size_t), value :: bytes
            integer(c_int), value :: rows, width
            type(c_ptr), intent(out) :: weights
        end function
        integer(c_int) function fh_f16_destroy(weights) bind(C, name='fortai_hip_f16_weights_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: weights
        end function
        integer(c_int) function fh_buffer_create(context, bytes, buffer) &
                bind(C, name='fortai_hip_q8_device_buffer_create')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context
            integer(c_size_t), value :: bytes
            type(c_ptr), intent(out) :: buffer
        end function
        integer(c_int) function fh_buffer_destroy(context, buffer) &
                bind(C, name='fortai_hip_q8_device_buffer_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: context, buffer
        end function
        integer(c_int) function fh_buffer_upload(context, buffer, host, bytes) &
                bind(C, name='fortai_hip_q8_device_buffer_upload_ptr')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, buffer, host
            integer(c_size_t), value :: bytes
        end function
        integer(c_int) function fh_buffer_download(context, host, buffer, bytes) &
                bind(C, name='fortai_hip_q8_device_buffer_download')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, host, buffer
            integer(c_size_t), value :: bytes
        end function
        integer(c_int) function fh_matvec_resident(context, weights, activation, output, kernel_ms) &
                bind(C, name='fortai_hip_q8_matvec_resident')
            import :: c_float, c_int, c_ptr
            type(c_ptr), value :: context, weights, activation, output
            real(c_float), intent(out) :: kernel_ms
        end function
        integer(c_int) function fh_matvec_device_f32(context, weights, activation, n_in, output, n_out) &
                bind(C, name='fortai_hip_q8_matvec_device_f32')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, weights, activation, output
            integer(c_size_t), value :: n_in, n_out
        end function
        integer(c_int) function fh_embedding(context, weights, token, output, n_out) &
                bind(C, name='fortai_hip_qwen35_embedding_device')
            import :: c_int, c_int64_t, c_ptr, c_size_t
            type(c_ptr), value :: context, weights, output
            integer(c_int64_t), value :: token
            integer(c_size_t), value :: n_out
        end function
        integer(c_int) function fh_copy(context, input, output, bytes) bind(C, name='fortai_hip_qwen35_copy_device')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, input, output
            integer(c_size_t), value :: bytes
        end function
        integer(c_int) function fh_add(context, left, right, output, n) bind(C, name='fortai_hip_qwen35_add_device')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, left, right, output
            integer(c_size_t), value :: n
        end function
        integer(c_int) function fh_rms_norm(context, input, weights, output, n, eps) &
                bind(C, name='fortai_hip_qwen35_rms_norm_device')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, input, weights, output
            integer(c_size_t), value :: n
            real(c_float), value :: eps
        end function
        integer(c_int) function fh_matvec_host(context, weights, act, act_bytes, out, out_bytes, ms) &
                bind(C, name='fortai_hip_q8_matvec_host')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, weights, act, out
            integer(c_size_t), value :: act_bytes, out_bytes
            real(c_float), intent(out) :: ms
        end function
        integer(c_int) function fh_matvec_host_pair(context, w1, w2, act, act_bytes, o1, b1, o2, b2, ms) &
                bind(C, name='fortai_hip_q8_matvec_host_pair')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, w1, w2, act, o1, o2
            integer(c_size_t), value :: act_bytes, b1, b2
            real(c_float), intent(out) :: ms
        end function
        integer(c_int) function fh_matvec_host_triplet(context, w1, w2, w3, act, act_bytes, o1, b1, o2, b2, &
                o3, b3, ms) bind(C, name='fortai_hip_q8_matvec_host_triplet')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, w1, w2, w3, act, o1, o2, o3
            integer(c_size_t), value :: act_bytes, b1, b2, b3
            real(c_float), intent(out) :: ms
        end function
        integer(c_int) function fh_matvec_host_contiguous(context, w1, w2, w3, act, act_bytes, out, out_bytes, &
                ms) bind(C, name='fortai_hip_q8_matvec_host_triplet_contiguous')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, w1, w2, w3, act, out
            integer(c_size_t), value :: act_bytes, out_bytes
            real(c_float), intent(out) :: ms
        end function
        integer(c_int) function fh_ffn_host(context, gate, up, down, act, act_bytes, out, out_bytes, ms) &
                bind(C, name='fortai_hip_q8_ffn_host')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, gate, up, down, act, out
            integer(c_size_t), value :: act_bytes, out_bytes
            real(c_float), intent(out) :: ms
        end function
        integer(c_int) function fh_ffn_device(context, gate, up, down, act, n_in, out, n_out) &
                bind(C, name='fortai_hip_q8_ffn_device')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, gate, up, down, act, out
            integer(c_size_t), value :: n_in, n_out
        end function
        integer(c_int) function fh_recurrent_create(context, qkv, gate, alpha, beta, output, conv, conv_bytes, &
                conv_size, conv_kernel, ssm_a, a_bytes, ssm_dt, dt_bytes, ssm_norm, norm_bytes, state_size, &
                key_heads, value_heads, head_size, inner_size, eps, layer) &
                bind(C, name='fortai_hip_qwen35_recurrent_create')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, qkv, gate, alpha, beta, output, conv, ssm_a, ssm_dt, ssm_norm
            integer(c_size_t), value :: conv_bytes, a_bytes, dt_bytes, norm_bytes
            integer(c_int), value :: conv_size, conv_kernel, state_size, key_heads, value_heads
            integer(c_int), value :: head_size, inner_size
            real(c_float), value :: eps
            type(c_ptr), intent(out) :: layer
        end function
        integer(c_int) function fh_recurrent_destroy(layer) bind(C, name='fortai_hip_qwen35_recurrent_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: layer
        end function
        integer(c_int) function fh_recurrent_reset(layer) bind(C, name='fortai_hip_qwen35_recurrent_reset')
            import :: c_int, c_ptr
            type(c_ptr), value :: layer
        end function
        integer(c_int) function fh_recurrent_run(layer, act, act_bytes, out, out_bytes, ms) &
                bind(C, name='fortai_hip_qwen35_recurrent_run')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: layer, act, out
            integer(c_size_t), value :: act_bytes, out_bytes
            real(c_float), intent(out) :: ms
        end function
        integer(c_int) function fh_recurrent_run_device(layer, act, n_in, out, n_out) &
                bind(C, name='fortai_hip_qwen35_recurrent_run_device')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: layer, act, out
            integer(c_size_t), value :: n_in, n_out
        end function
        integer(c_int) function fh_attention_create(context, wq, wk, wv, wo, q_norm, q_norm_bytes, k_norm, &
                k_norm_bytes, heads, kv_heads, head_size, value_size, max_context, rope_dim, rope_base, eps, &
                layer) bind(C, name='fortai_hip_qwen35_attention_create')
            import :: c_float, c_int, c_ptr, c_size_t
            type(c_ptr), value :: context, wq, wk, wv, wo, q_norm, k_norm
            integer(c_size_t), value :: q_norm_bytes, k_norm_bytes
            integer(c_int), value :: heads, kv_heads, head_size, value_size, max_context, rope_dim
            real(c_float), value :: rope_base, eps
            type(c_ptr), intent(out) :: layer
        end function
        integer(c_int) function fh_attention_destroy(layer) bind(C, name='fortai_hip_qwen35_attention_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: layer
        end function
        integer(c_int) function fh_attention_reset(layer) bind(C, name='fortai_hip_qwen35_attention_reset')
            import :: c_int, c_ptr
            type(c_ptr), value :: layer
        end function
        integer(c_int) function fh_attention_run_device(layer, act, n_in, position, out, n_out) &
                bind(C, name='fortai_hip_qwen35_attention_run_device')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: layer, act, out
            integer(c_size_t), value :: n_in, n_out
            integer(c_int), value :: position
        end function
        integer(c_int) function fh_decoder_create(context, layer_count, recurrent, attention, ffn_gate, ffn_up, &
                ffn_down, attn_norm, post_norm, output_norm, hidden, emb16, emb8, out16, out8, max_context, &
                eps, decoder) bind(C, name='fortai_hip_qwen35_decoder_create')
            import :: c_float, c_int, c_ptr
            type(c_ptr), value :: context
            integer(c_int), value :: layer_count, hidden, max_context
            type(c_ptr), intent(in) :: recurrent(*), attention(*), ffn_gate(*), ffn_up(*), ffn_down(*)
            type(c_ptr), intent(in) :: attn_norm(*), post_norm(*)
            type(c_ptr), value :: output_norm, emb16, emb8, out16, out8
            real(c_float), value :: eps
            type(c_ptr), intent(out) :: decoder
        end function
        integer(c_int) function fh_decoder_destroy(decoder) bind(C, name='fortai_hip_qwen35_decoder_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: decoder
        end function
        integer(c_int) function fh_decoder_reset(decoder) bind(C, name='fortai_hip_qwen35_decoder_reset')
            import :: c_int, c_ptr
            type(c_ptr), value :: decoder
        end function
        integer(c_int) function fh_decoder_forward(decoder, token, position, logits, next_token) &
                bind(C, name='fortai_hip_qwen35_decoder_forward')
            import :: c_int, c_int64_t, c_ptr
            type(c_ptr), value :: decoder, logits, next_token
            integer(c_int64_t), value :: token
            integer(c_int), value :: position
        end function
        integer(c_int) function fh_decoder_generate(decoder, token, position, steps, trace) &
                bind(C, name='fortai_hip_qwen35_decoder_generate')
            import :: c_int, c_int64_t, c_ptr
            type(c_ptr), value :: decoder, trace
            integer(c_int64_t), value :: token
            integer(c_int), value :: position, steps
        end function
        integer(c_int) function fh_batch_create(context, batch, layer_count, recurrent, attention, ffn_gate, &
                ffn_up, ffn_down, attn_norm, post_norm, output_norm, hidden, emb16, emb8, out16, out8, &
                max_context, eps, decoder) bind(C, name='fortai_hip_qwen35_batch_create')
            import :: c_float, c_int, c_ptr
            type(c_ptr), value :: context
            integer(c_int), value :: batch, layer_count, hidden, max_context
            type(c_ptr), intent(in) :: recurrent(*), attention(*), ffn_gate(*), ffn_up(*), ffn_down(*)
            type(c_ptr), intent(in) :: attn_norm(*), post_norm(*)
            type(c_ptr), value :: output_norm, emb16, emb8, out16, out8
            real(c_float), value :: eps
            type(c_ptr), intent(out) :: decoder
        end function
        integer(c_int) function fh_batch_destroy(decoder) bind(C, name='fortai_hip_qwen35_batch_destroy')
            import :: c_int, c_ptr
            type(c_ptr), value :: decoder
        end function
        integer(c_int) function fh_batch_reset(decoder) bind(C, name='fortai_hip_qwen35_batch_reset')
            import :: c_int, c_ptr
            type(c_ptr), value :: decoder
        end function
        integer(c_int) function fh_batch_prefill(decoder, tokens, t, next_tokens, logits, kernel_ms) &
                bind(C, name='fortai_hip_qwen35_batch_prefill')
            import :: c_int, c_ptr
            type(c_ptr), value :: decoder, tokens, next_tokens, logits, kernel_ms
            integer(c_int), value :: t
        end function
        integer(c_int) function fh_batch_generate(decoder, tokens, positions, steps, trace) &
                bind(C, name='fortai_hip_qwen35_batch_generate')
            import :: c_int, c_ptr
            type(c_ptr), value :: decoder, tokens, positions, trace
            integer(c_int), value :: steps
        end function
        integer(c_int) function fh_decoder_plan(decoder, buffer, bytes, needed) &
                bind(C, name='fortai_hip_qwen35_decoder_plan')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: decoder, buffer
            integer(c_size_t), value :: bytes
            integer(c_size_t), intent(out) :: needed
        end function
        integer(c_int) function fh_batch_plan(decoder, prefill, buffer, bytes, needed) &
                bind(C, name='fortai_hip_qwen35_batch_plan')
            import :: c_int, c_ptr, c_size_t
            type(c_ptr), value :: decoder
            integer(c_int), value :: prefill
            type(c_ptr), value :: buffer
            integer(c_size_t), value :: bytes
            integer(c_size_t), intent(out) :: needed
        end function
        integer(c_int) function c_strlen(s) bind(C, name='strlen')
            import :: c_int, c_ptr
            type(c_ptr), value :: s
        end function
    end interface

contains

    ! ---- helpers ---------------------------------------------------------------

    ! Detailed text of the context's last failure (empty if none).
    function error_text(context) result(text)
        type(c_ptr), intent(in) :: context
        character(len=:), allocatable :: text
        type(c_ptr) :: raw
        character(kind=c_char), pointer :: chars(:)
        integer :: n, i

        text = ''
        raw = fh_last_error(context)
        if (.not. c_associated(raw)) return
        n = c_strlen(raw)
        if (n <= 0) return
        call c_f_pointer(raw, chars, [n])
        allocate (character(len=n) :: text)
        do i = 1, n
            text(i:i) = chars(i)
        end do
    end function error_text

    ! Map a C return code onto the status: non-zero -> FORTAI_UNSUPPORTED with
    ! the operation name and the library's message.
    subroutine settle(code, context, what, stat)
        integer(c_int), intent(in) :: code
        type(c_ptr), intent(in) :: context
        character(len=*), intent(in) :: what
        type(status_t), intent(inout) :: stat
        character(len=:), allocatable :: detail

        if (code == FORTAI_HIP_OK) return
        detail = ''
        if (c_associated(context)) detail = error_text(context)
        if (len(detail) > 0) then
            call stat%set(FORTAI_UNSUPPORTED, 'HIP ' // what // ' failed: ' // detail)
        else
            call stat%set(FORTAI_UNSUPPORTED, 'HIP ' // what // ' failed')
        end if
    end subroutine settle

    logical function live(handle)
        type(c_ptr), intent(in) :: handle
        live = c_associated(handle)
    end function live

    integer(c_size_t) function real_bytes(values)
        real(c_float), intent(in) :: values(:)
        real_bytes = int(size(values), c_size_t) * 4_c_size_t
    end function real_bytes

    ! ---- context ---------------------------------------------------------------

    subroutine context_create(self, device, stat)
        class(hip_q8_context_t), intent(inout) :: self
        integer, intent(in) :: device
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (live(self%handle)) call self%destroy(stat)
        code = fh_context_create(int(device, c_int), self%handle)
        if (code /= FORTAI_HIP_OK) then
            self%handle = c_null_ptr
            call stat%set(FORTAI_UNSUPPORTED, 'HIP Q8 context creation failed')
        end if
    end subroutine context_create

    subroutine context_destroy(self, stat)
        class(hip_q8_context_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle)) return
        code = fh_context_call(self%handle)
        self%handle = c_null_ptr
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, 'HIP Q8 context destruction failed')
    end subroutine context_destroy

    subroutine context_set_position(self, position, stat)
        class(hip_q8_context_t), intent(in) :: self
        integer, intent(in) :: position
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. position < 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device position')
            return
        end if
        call settle(fh_set_position(self%handle, int(position, c_int)), self%handle, 'device position update', stat)
    end subroutine context_set_position

    subroutine context_capture_begin(self, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP graph context')
            return
        end if
        call settle(fh_capture_begin(self%handle), self%handle, 'graph capture begin', stat)
    end subroutine context_capture_begin

    subroutine context_capture_end(self, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP graph context')
            return
        end if
        call settle(fh_capture_end(self%handle), self%handle, 'graph capture end', stat)
    end subroutine context_capture_end

    subroutine context_graph_launch(self, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP graph context')
            return
        end if
        call settle(fh_graph_launch(self%handle), self%handle, 'graph launch', stat)
    end subroutine context_graph_launch

    subroutine context_synchronize(self, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP context')
            return
        end if
        call settle(fh_synchronize(self%handle), self%handle, 'stream synchronize', stat)
    end subroutine context_synchronize

    subroutine context_allocate_buffer(self, bytes, buffer, stat)
        class(hip_q8_context_t), intent(in) :: self
        integer(c_size_t), intent(in) :: bytes
        type(c_ptr), intent(out) :: buffer
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        buffer = c_null_ptr
        if (.not. live(self%handle) .or. bytes <= 0_c_size_t) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device buffer')
            return
        end if
        code = fh_buffer_create(self%handle, bytes, buffer)
        if (code /= FORTAI_HIP_OK) buffer = c_null_ptr
        call settle(code, self%handle, 'device buffer allocation', stat)
    end subroutine context_allocate_buffer

    subroutine context_free_buffer(self, buffer, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(c_ptr), intent(inout) :: buffer
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle) .or. .not. live(buffer)) return
        code = fh_buffer_destroy(self%handle, buffer)
        buffer = c_null_ptr
        call settle(code, self%handle, 'device buffer release', stat)
    end subroutine context_free_buffer

    subroutine context_upload(self, buffer, host_data, bytes, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(c_ptr), intent(in) :: buffer
        integer(c_int8_t), contiguous, target, intent(in) :: host_data(:)
        integer(c_size_t), intent(in) :: bytes
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. .not. live(buffer) .or. size(host_data) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device upload')
            return
        end if
        call settle(fh_buffer_upload(self%handle, buffer, c_loc(host_data), bytes), self%handle, &
            'device upload', stat)
    end subroutine context_upload

    subroutine context_upload_real(self, buffer, host_data, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(c_ptr), intent(in) :: buffer
        real(c_float), contiguous, target, intent(in) :: host_data(:)
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. .not. live(buffer) .or. size(host_data) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP real device upload')
            return
        end if
        call settle(fh_buffer_upload(self%handle, buffer, c_loc(host_data), real_bytes(host_data)), &
            self%handle, 'real device upload', stat)
    end subroutine context_upload_real

    subroutine context_download(self, buffer, host_data, bytes, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(c_ptr), intent(in) :: buffer
        integer(c_int8_t), contiguous, target, intent(out) :: host_data(:)
        integer(c_size_t), intent(in) :: bytes
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. .not. live(buffer) .or. size(host_data) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device download')
            return
        end if
        call settle(fh_buffer_download(self%handle, c_loc(host_data), buffer, bytes), self%handle, &
            'device download', stat)
    end subroutine context_download

    subroutine context_download_real(self, buffer, host_data, stat)
        class(hip_q8_context_t), intent(in) :: self
        type(c_ptr), intent(in) :: buffer
        real(c_float), contiguous, target, intent(out) :: host_data(:)
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. .not. live(buffer) .or. size(host_data) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP real device download')
            return
        end if
        call settle(fh_buffer_download(self%handle, c_loc(host_data), buffer, real_bytes(host_data)), &
            self%handle, 'real device download', stat)
    end subroutine context_download_real

    function context_last_error(self) result(message)
        class(hip_q8_context_t), intent(in) :: self
        character(len=:), allocatable :: message

        if (.not. live(self%handle)) then
            message = 'HIP Q8 context is not initialized'
            return
        end if
        message = error_text(self%handle)
        if (len(message) == 0) message = 'no HIP backend error recorded'
    end function context_last_error

    ! ---- weights -----------------------------------------------------------------

    subroutine q8_weights_upload(self, context, host_weights, weight_bytes, rows, width, stat)
        class(hip_q8_weights_t), intent(inout) :: self
        class(hip_q8_context_t), intent(in) :: context
        integer(c_int8_t), contiguous, target, intent(in) :: host_weights(:)
        integer(c_size_t), intent(in) :: weight_bytes
        integer, intent(in) :: rows, width
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(context%handle) .or. size(host_weights) <= 0 .or. rows <= 0 .or. width <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 weight upload')
            return
        end if
        if (live(self%handle)) call self%destroy(stat)
        code = fh_weights_upload(context%handle, c_loc(host_weights), weight_bytes, int(rows, c_int), &
            int(width, c_int), self%handle)
        if (code /= FORTAI_HIP_OK) self%handle = c_null_ptr
        call settle(code, context%handle, 'Q8 weight upload', stat)
    end subroutine q8_weights_upload

    subroutine q8_weights_destroy(self, stat)
        class(hip_q8_weights_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle)) return
        code = fh_weights_destroy(self%handle)
        self%handle = c_null_ptr
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, 'HIP Q8 weight destruction failed')
    end subroutine q8_weights_destroy

    ! Bytes of the resident planes of a rows x width Q8_0 matrix (0 if the
    ! shape is invalid): the size of a pack record.
    function hip_q8_pack_bytes(rows, width) result(bytes)
        integer, intent(in) :: rows, width
        integer(c_size_t) :: bytes

        bytes = 0_c_size_t
        if (rows <= 0 .or. width <= 0) return
        bytes = fh_pack_bytes(int(rows, c_int), int(width, c_int))
    end function hip_q8_pack_bytes

    ! Copy the resident planes to host memory (synchronous); host_planes must
    ! hold hip_q8_pack_bytes(rows, width) bytes.
    subroutine q8_weights_pack(self, host_planes, stat)
        class(hip_q8_weights_t), intent(in) :: self
        integer(c_int8_t), contiguous, target, intent(inout) :: host_planes(:)
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle) .or. size(host_planes) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 weight pack')
            return
        end if
        code = fh_weights_pack(self%handle, c_loc(host_planes), int(size(host_planes), c_size_t))
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, &
            'HIP Q8 weight pack failed (buffer smaller than the planes, or a device error)')
    end subroutine q8_weights_pack

    ! Create the resident matrix from planes written by pack (no repack).
    subroutine q8_weights_upload_packed(self, context, host_planes, rows, width, stat)
        class(hip_q8_weights_t), intent(inout) :: self
        class(hip_q8_context_t), intent(in) :: context
        integer(c_int8_t), contiguous, target, intent(in) :: host_planes(:)
        integer, intent(in) :: rows, width
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(context%handle) .or. rows <= 0 .or. width <= 0 .or. &
                int(size(host_planes), c_size_t) < hip_q8_pack_bytes(rows, width) .or. &
                hip_q8_pack_bytes(rows, width) == 0_c_size_t) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 packed weight upload')
            return
        end if
        if (live(self%handle)) call self%destroy(stat)
        code = fh_weights_upload_packed(context%handle, c_loc(host_planes), int(size(host_planes), c_size_t), &
            int(rows, c_int), int(width, c_int), self%handle)
        if (code /= FORTAI_HIP_OK) self%handle = c_null_ptr
        call settle(code, context%handle, 'Q8 packed weight upload', stat)
    end subroutine q8_weights_upload_packed

    subroutine f16_weights_upload(self, context, host_weights, weight_bytes, rows, width, stat)
        class(hip_f16_weights_t), intent(inout) :: self
        class(hip_q8_context_t), intent(in) :: context
        integer(c_int8_t), contiguous, target, intent(in) :: host_weights(:)
        integer(c_size_t), intent(in) :: weight_bytes
        integer, intent(in) :: rows, width
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(context%handle) .or. size(host_weights) <= 0 .or. rows <= 0 .or. width <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP F16 weight upload')
            return
        end if
        if (live(self%handle)) call self%destroy(stat)
        code = fh_f16_upload(context%handle, c_loc(host_weights), weight_bytes, int(rows, c_int), &
            int(width, c_int), self%handle)
        if (code /= FORTAI_HIP_OK) self%handle = c_null_ptr
        call settle(code, context%handle, 'F16 weight upload', stat)
    end subroutine f16_weights_upload

    subroutine f16_weights_destroy(self, stat)
        class(hip_f16_weights_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle)) return
        code = fh_f16_destroy(self%handle)
        self%handle = c_null_ptr
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, 'HIP F16 weight destruction failed')
    end subroutine f16_weights_destroy

    ! ---- resident (device-pointer) operations --------------------------------

    subroutine hip_q8_matvec_resident(context, weights, activation, output, kernel_ms, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: weights
        type(c_ptr), intent(in) :: activation, output
        real(c_float), intent(out) :: kernel_ms
        type(status_t), intent(out) :: stat

        call stat%clear()
        kernel_ms = 0.0_c_float
        if (.not. (live(context%handle) .and. live(weights%handle) .and. live(activation) .and. &
                live(output))) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 resident matvec')
            return
        end if
        call settle(fh_matvec_resident(context%handle, weights%handle, activation, output, kernel_ms), &
            context%handle, 'Q8 resident matvec', stat)
    end subroutine hip_q8_matvec_resident

    subroutine hip_q8_matvec_device_f32(context, weights, activation, activation_elements, &
            output, output_elements, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: weights
        type(c_ptr), intent(in) :: activation, output
        integer(c_size_t), intent(in) :: activation_elements, output_elements
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(context%handle) .and. live(weights%handle) .and. live(activation) .and. &
                live(output)) .or. activation_elements <= 0 .or. output_elements <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device F32 matvec')
            return
        end if
        call settle(fh_matvec_device_f32(context%handle, weights%handle, activation, activation_elements, &
            output, output_elements), context%handle, 'device F32 matvec', stat)
    end subroutine hip_q8_matvec_device_f32

    subroutine hip_qwen35_embedding_device(context, weights, token_id, output, output_elements, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: weights
        integer(c_int64_t), intent(in) :: token_id
        type(c_ptr), intent(in) :: output
        integer(c_size_t), intent(in) :: output_elements
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(context%handle) .and. live(weights%handle) .and. live(output)) .or. &
                token_id < 0 .or. output_elements <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP embedding lookup')
            return
        end if
        call settle(fh_embedding(context%handle, weights%handle, token_id, output, output_elements), &
            context%handle, 'embedding lookup', stat)
    end subroutine hip_qwen35_embedding_device

    subroutine hip_qwen35_copy_device(context, device_input, device_output, bytes, stat)
        class(hip_q8_context_t), intent(in) :: context
        type(c_ptr), intent(in) :: device_input, device_output
        integer(c_size_t), intent(in) :: bytes
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(context%handle) .and. live(device_input) .and. live(device_output)) .or. &
                bytes <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device copy')
            return
        end if
        call settle(fh_copy(context%handle, device_input, device_output, bytes), context%handle, &
            'device copy', stat)
    end subroutine hip_qwen35_copy_device

    subroutine hip_qwen35_add_device(context, device_left, device_right, device_output, elements, stat)
        class(hip_q8_context_t), intent(in) :: context
        type(c_ptr), intent(in) :: device_left, device_right, device_output
        integer(c_size_t), intent(in) :: elements
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(context%handle) .and. live(device_left) .and. live(device_right) .and. &
                live(device_output)) .or. elements <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device add')
            return
        end if
        call settle(fh_add(context%handle, device_left, device_right, device_output, elements), &
            context%handle, 'device add', stat)
    end subroutine hip_qwen35_add_device

    subroutine hip_qwen35_rms_norm_device(context, device_input, device_weights, device_output, &
            elements, epsilon, stat)
        class(hip_q8_context_t), intent(in) :: context
        type(c_ptr), intent(in) :: device_input, device_weights, device_output
        integer(c_size_t), intent(in) :: elements
        real(c_float), intent(in) :: epsilon
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(context%handle) .and. live(device_input) .and. live(device_weights) .and. &
                live(device_output)) .or. elements <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device RMS norm')
            return
        end if
        call settle(fh_rms_norm(context%handle, device_input, device_weights, device_output, elements, &
            epsilon), context%handle, 'device RMS norm', stat)
    end subroutine hip_qwen35_rms_norm_device

    ! ---- host-controlled operations (host Q8_0 activation in, host f32 out) ----

    subroutine hip_q8_matvec_host(context, weights, activation, activation_bytes, output, &
            output_bytes, elapsed_ms, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: weights
        integer(c_int8_t), contiguous, target, intent(in) :: activation(:)
        integer(c_size_t), intent(in) :: activation_bytes, output_bytes
        real(c_float), contiguous, target, intent(out) :: output(:)
        real(c_float), intent(out) :: elapsed_ms
        type(status_t), intent(out) :: stat

        call stat%clear()
        elapsed_ms = 0.0_c_float
        if (.not. (live(context%handle) .and. live(weights%handle)) .or. size(activation) <= 0 .or. &
                size(output) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 matvec')
            return
        end if
        call settle(fh_matvec_host(context%handle, weights%handle, c_loc(activation), activation_bytes, &
            c_loc(output), output_bytes, elapsed_ms), context%handle, 'Q8 matvec', stat)
    end subroutine hip_q8_matvec_host

    subroutine hip_q8_matvec_host_pair(context, first_weights, second_weights, activation, &
            activation_bytes, first_output, first_output_bytes, second_output, second_output_bytes, &
            elapsed_ms, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: first_weights, second_weights
        integer(c_int8_t), contiguous, target, intent(in) :: activation(:)
        integer(c_size_t), intent(in) :: activation_bytes, first_output_bytes, second_output_bytes
        real(c_float), contiguous, target, intent(out) :: first_output(:), second_output(:)
        real(c_float), intent(out) :: elapsed_ms
        type(status_t), intent(out) :: stat

        call stat%clear()
        elapsed_ms = 0.0_c_float
        if (.not. (live(context%handle) .and. live(first_weights%handle) .and. &
                live(second_weights%handle)) .or. size(activation) <= 0 .or. size(first_output) <= 0 .or. &
                size(second_output) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 paired matvec')
            return
        end if
        call settle(fh_matvec_host_pair(context%handle, first_weights%handle, second_weights%handle, &
            c_loc(activation), activation_bytes, c_loc(first_output), first_output_bytes, &
            c_loc(second_output), second_output_bytes, elapsed_ms), context%handle, 'Q8 paired matvec', stat)
    end subroutine hip_q8_matvec_host_pair

    subroutine hip_q8_matvec_host_triplet(context, first_weights, second_weights, third_weights, &
            activation, activation_bytes, first_output, first_output_bytes, second_output, &
            second_output_bytes, third_output, third_output_bytes, elapsed_ms, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: first_weights, second_weights, third_weights
        integer(c_int8_t), contiguous, target, intent(in) :: activation(:)
        integer(c_size_t), intent(in) :: activation_bytes
        integer(c_size_t), intent(in) :: first_output_bytes, second_output_bytes, third_output_bytes
        real(c_float), contiguous, target, intent(out) :: first_output(:), second_output(:), third_output(:)
        real(c_float), intent(out) :: elapsed_ms
        type(status_t), intent(out) :: stat

        call stat%clear()
        elapsed_ms = 0.0_c_float
        if (.not. (live(context%handle) .and. live(first_weights%handle) .and. &
                live(second_weights%handle) .and. live(third_weights%handle)) .or. size(activation) <= 0 .or. &
                size(first_output) <= 0 .or. size(second_output) <= 0 .or. size(third_output) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 triplet matvec')
            return
        end if
        call settle(fh_matvec_host_triplet(context%handle, first_weights%handle, second_weights%handle, &
            third_weights%handle, c_loc(activation), activation_bytes, c_loc(first_output), &
            first_output_bytes, c_loc(second_output), second_output_bytes, c_loc(third_output), &
            third_output_bytes, elapsed_ms), context%handle, 'Q8 triplet matvec', stat)
    end subroutine hip_q8_matvec_host_triplet

    subroutine hip_q8_matvec_host_triplet_contiguous(context, first_weights, second_weights, &
            third_weights, activation, activation_bytes, host_output, host_output_bytes, elapsed_ms, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: first_weights, second_weights, third_weights
        integer(c_int8_t), contiguous, target, intent(in) :: activation(:)
        integer(c_size_t), intent(in) :: activation_bytes, host_output_bytes
        real(c_float), contiguous, target, intent(out) :: host_output(:)
        real(c_float), intent(out) :: elapsed_ms
        type(status_t), intent(out) :: stat

        call stat%clear()
        elapsed_ms = 0.0_c_float
        if (.not. (live(context%handle) .and. live(first_weights%handle) .and. &
                live(second_weights%handle) .and. live(third_weights%handle)) .or. size(activation) <= 0 .or. &
                size(host_output) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 contiguous triplet matvec')
            return
        end if
        call settle(fh_matvec_host_contiguous(context%handle, first_weights%handle, second_weights%handle, &
            third_weights%handle, c_loc(activation), activation_bytes, c_loc(host_output), &
            host_output_bytes, elapsed_ms), context%handle, 'Q8 contiguous triplet matvec', stat)
    end subroutine hip_q8_matvec_host_triplet_contiguous

    subroutine hip_q8_ffn_host(context, gate_weights, up_weights, down_weights, host_activation, &
            activation_bytes, host_output, output_bytes, elapsed_ms, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: gate_weights, up_weights, down_weights
        integer(c_int8_t), contiguous, target, intent(in) :: host_activation(:)
        integer(c_size_t), intent(in) :: activation_bytes, output_bytes
        real(c_float), contiguous, target, intent(out) :: host_output(:)
        real(c_float), intent(out) :: elapsed_ms
        type(status_t), intent(out) :: stat

        call stat%clear()
        elapsed_ms = 0.0_c_float
        if (.not. (live(context%handle) .and. live(gate_weights%handle) .and. live(up_weights%handle) .and. &
                live(down_weights%handle)) .or. size(host_activation) <= 0 .or. size(host_output) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Q8 FFN')
            return
        end if
        call settle(fh_ffn_host(context%handle, gate_weights%handle, up_weights%handle, down_weights%handle, &
            c_loc(host_activation), activation_bytes, c_loc(host_output), output_bytes, elapsed_ms), &
            context%handle, 'Q8 FFN', stat)
    end subroutine hip_q8_ffn_host

    subroutine hip_q8_ffn_device(context, gate_weights, up_weights, down_weights, device_activation, &
            activation_elements, device_output, output_elements, stat)
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: gate_weights, up_weights, down_weights
        type(c_ptr), intent(in) :: device_activation, device_output
        integer(c_size_t), intent(in) :: activation_elements, output_elements
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(context%handle) .and. live(gate_weights%handle) .and. live(up_weights%handle) .and. &
                live(down_weights%handle) .and. live(device_activation) .and. live(device_output)) .or. &
                activation_elements <= 0 .or. output_elements <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP device Q8 FFN')
            return
        end if
        call settle(fh_ffn_device(context%handle, gate_weights%handle, up_weights%handle, down_weights%handle, &
            device_activation, activation_elements, device_output, output_elements), context%handle, &
            'device Q8 FFN', stat)
    end subroutine hip_q8_ffn_device

    ! ---- Gated DeltaNet layer ----------------------------------------------------

    subroutine recurrent_create(self, context, qkv_weights, gate_weights, alpha_weights, &
            beta_weights, output_weights, conv_weights, conv_weight_bytes, conv_size, conv_kernel, &
            ssm_a, ssm_a_bytes, ssm_dt, ssm_dt_bytes, ssm_norm, ssm_norm_bytes, state_size, &
            key_heads, value_heads, head_size, inner_size, norm_epsilon, stat)
        class(hip_qwen35_recurrent_t), intent(inout) :: self
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: qkv_weights, gate_weights, alpha_weights
        class(hip_q8_weights_t), intent(in) :: beta_weights, output_weights
        integer(c_int8_t), contiguous, target, intent(in) :: conv_weights(:), ssm_a(:), ssm_dt(:), ssm_norm(:)
        integer(c_size_t), intent(in) :: conv_weight_bytes, ssm_a_bytes, ssm_dt_bytes, ssm_norm_bytes
        integer, intent(in) :: conv_size, conv_kernel, state_size, key_heads, value_heads
        integer, intent(in) :: head_size, inner_size
        real(c_float), intent(in) :: norm_epsilon
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. (live(context%handle) .and. live(qkv_weights%handle) .and. live(gate_weights%handle) .and. &
                live(alpha_weights%handle) .and. live(beta_weights%handle) .and. &
                live(output_weights%handle)) .or. min(size(conv_weights), size(ssm_a), size(ssm_dt), &
                size(ssm_norm)) <= 0 .or. min(conv_size, conv_kernel, state_size, key_heads, value_heads, &
                head_size, inner_size) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen recurrent layer arguments')
            return
        end if
        if (live(self%handle)) call self%destroy(stat)
        code = fh_recurrent_create(context%handle, qkv_weights%handle, gate_weights%handle, &
            alpha_weights%handle, beta_weights%handle, output_weights%handle, c_loc(conv_weights), &
            conv_weight_bytes, int(conv_size, c_int), int(conv_kernel, c_int), c_loc(ssm_a), ssm_a_bytes, &
            c_loc(ssm_dt), ssm_dt_bytes, c_loc(ssm_norm), ssm_norm_bytes, int(state_size, c_int), &
            int(key_heads, c_int), int(value_heads, c_int), int(head_size, c_int), int(inner_size, c_int), &
            norm_epsilon, self%handle)
        if (code /= FORTAI_HIP_OK) then
            self%handle = c_null_ptr
            self%context = c_null_ptr
        else
            self%context = context%handle
        end if
        call settle(code, context%handle, 'Qwen recurrent layer creation', stat)
    end subroutine recurrent_create

    subroutine recurrent_destroy(self, stat)
        class(hip_qwen35_recurrent_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle)) return
        code = fh_recurrent_destroy(self%handle)
        self%handle = c_null_ptr
        self%context = c_null_ptr
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, 'HIP Qwen recurrent layer destruction failed')
    end subroutine recurrent_destroy

    subroutine recurrent_reset(self, stat)
        class(hip_qwen35_recurrent_t), intent(in) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) return
        call settle(fh_recurrent_reset(self%handle), self%context, 'Qwen recurrent state reset', stat)
    end subroutine recurrent_reset

    subroutine recurrent_run(self, host_activation, activation_bytes, host_output, &
            output_bytes, elapsed_ms, stat)
        class(hip_qwen35_recurrent_t), intent(in) :: self
        integer(c_int8_t), contiguous, target, intent(in) :: host_activation(:)
        integer(c_size_t), intent(in) :: activation_bytes, output_bytes
        real(c_float), contiguous, target, intent(out) :: host_output(:)
        real(c_float), intent(out) :: elapsed_ms
        type(status_t), intent(out) :: stat

        call stat%clear()
        elapsed_ms = 0.0_c_float
        if (.not. live(self%handle) .or. size(host_activation) <= 0 .or. size(host_output) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen recurrent execution arguments')
            return
        end if
        call settle(fh_recurrent_run(self%handle, c_loc(host_activation), activation_bytes, &
            c_loc(host_output), output_bytes, elapsed_ms), self%context, 'Qwen recurrent execution', stat)
    end subroutine recurrent_run

    subroutine recurrent_run_device(self, device_activation, activation_elements, &
            device_output, output_elements, stat)
        class(hip_qwen35_recurrent_t), intent(in) :: self
        type(c_ptr), intent(in) :: device_activation, device_output
        integer(c_size_t), intent(in) :: activation_elements, output_elements
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(self%handle) .and. live(device_activation) .and. live(device_output)) .or. &
                activation_elements <= 0 .or. output_elements <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen recurrent device arguments')
            return
        end if
        call settle(fh_recurrent_run_device(self%handle, device_activation, activation_elements, &
            device_output, output_elements), self%context, 'Qwen recurrent device execution', stat)
    end subroutine recurrent_run_device

    ! ---- gated full-attention layer ------------------------------------------------

    subroutine attention_create(self, context, query_weights, key_weights, value_weights, &
            output_weights, query_norm, query_norm_bytes, key_norm, key_norm_bytes, heads, &
            key_value_heads, head_size, value_size, max_context, rope_dimension, rope_base, &
            norm_epsilon, stat)
        class(hip_qwen35_attention_t), intent(inout) :: self
        class(hip_q8_context_t), intent(in) :: context
        class(hip_q8_weights_t), intent(in) :: query_weights, key_weights, value_weights, output_weights
        integer(c_int8_t), contiguous, target, intent(in) :: query_norm(:), key_norm(:)
        integer(c_size_t), intent(in) :: query_norm_bytes, key_norm_bytes
        integer, intent(in) :: heads, key_value_heads, head_size, value_size, max_context, rope_dimension
        real(c_float), intent(in) :: rope_base, norm_epsilon
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. (live(context%handle) .and. live(query_weights%handle) .and. live(key_weights%handle) .and. &
                live(value_weights%handle) .and. live(output_weights%handle)) .or. &
                min(size(query_norm), size(key_norm)) <= 0 .or. min(heads, key_value_heads, head_size, &
                value_size, max_context, rope_dimension) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen attention layer arguments')
            return
        end if
        if (live(self%handle)) call self%destroy(stat)
        code = fh_attention_create(context%handle, query_weights%handle, key_weights%handle, &
            value_weights%handle, output_weights%handle, c_loc(query_norm), query_norm_bytes, c_loc(key_norm), &
            key_norm_bytes, int(heads, c_int), int(key_value_heads, c_int), int(head_size, c_int), &
            int(value_size, c_int), int(max_context, c_int), int(rope_dimension, c_int), rope_base, &
            norm_epsilon, self%handle)
        if (code /= FORTAI_HIP_OK) then
            self%handle = c_null_ptr
            self%context = c_null_ptr
        else
            self%context = context%handle
        end if
        call settle(code, context%handle, 'Qwen attention layer creation', stat)
    end subroutine attention_create

    subroutine attention_destroy(self, stat)
        class(hip_qwen35_attention_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle)) return
        code = fh_attention_destroy(self%handle)
        self%handle = c_null_ptr
        self%context = c_null_ptr
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, 'HIP Qwen attention layer destruction failed')
    end subroutine attention_destroy

    subroutine attention_reset(self, stat)
        class(hip_qwen35_attention_t), intent(inout) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) return
        call settle(fh_attention_reset(self%handle), self%context, 'Qwen attention cache reset', stat)
    end subroutine attention_reset

    subroutine attention_run_device(self, device_activation, activation_elements, position, &
            device_output, output_elements, stat)
        class(hip_qwen35_attention_t), intent(in) :: self
        type(c_ptr), intent(in) :: device_activation, device_output
        integer(c_size_t), intent(in) :: activation_elements, output_elements
        integer, intent(in) :: position
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. (live(self%handle) .and. live(device_activation) .and. live(device_output)) .or. &
                position < 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen attention execution arguments')
            return
        end if
        call settle(fh_attention_run_device(self%handle, device_activation, activation_elements, &
            int(position, c_int), device_output, output_elements), self%context, &
            'Qwen attention device execution', stat)
    end subroutine attention_run_device

    ! ---- fused decoder (one captured graph per token) ------------------------------

    ! Layer i uses recurrent(i) when its handle is set, else attention(i).
    ! attn_norm / post_norm are host fp32 [hidden, layers]; exactly one of
    ! embedding_f16 / embedding_q8 and one of output_f16 / output_q8 is set.
    subroutine decoder_create(self, context, recurrent, attention, ffn_gate, ffn_up, ffn_down, &
            attn_norm, post_norm, output_norm, embedding_f16, embedding_q8, output_f16, output_q8, &
            max_context, norm_epsilon, stat)
        class(hip_qwen35_decoder_t), intent(inout) :: self
        class(hip_q8_context_t), intent(in) :: context
        type(hip_qwen35_recurrent_t), intent(in) :: recurrent(:)
        type(hip_qwen35_attention_t), intent(in) :: attention(:)
        type(hip_q8_weights_t), intent(in) :: ffn_gate(:), ffn_up(:), ffn_down(:)
        real(c_float), contiguous, target, intent(in) :: attn_norm(:, :), post_norm(:, :), output_norm(:)
        type(hip_f16_weights_t), intent(in) :: embedding_f16, output_f16
        type(hip_q8_weights_t), intent(in) :: embedding_q8, output_q8
        integer, intent(in) :: max_context
        real(c_float), intent(in) :: norm_epsilon
        type(status_t), intent(out) :: stat
        type(c_ptr), allocatable :: rec(:), att(:), gate(:), up(:), down(:), an(:), pn(:)
        integer :: n, i
        integer(c_int) :: code

        call stat%clear()
        n = size(ffn_gate)
        if (.not. live(context%handle) .or. n <= 0 .or. size(recurrent) /= n .or. size(attention) /= n .or. &
                size(ffn_up) /= n .or. size(ffn_down) /= n .or. size(attn_norm, 2) /= n .or. &
                size(post_norm, 2) /= n .or. size(attn_norm, 1) /= size(output_norm) .or. &
                size(post_norm, 1) /= size(output_norm) .or. max_context <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen decoder arguments')
            return
        end if
        allocate (rec(n), att(n), gate(n), up(n), down(n), an(n), pn(n))
        do i = 1, n
            rec(i) = recurrent(i)%handle
            att(i) = attention(i)%handle
            gate(i) = ffn_gate(i)%handle
            up(i) = ffn_up(i)%handle
            down(i) = ffn_down(i)%handle
            an(i) = c_loc(attn_norm(1, i))
            pn(i) = c_loc(post_norm(1, i))
        end do
        if (live(self%handle)) call self%destroy(stat)
        code = fh_decoder_create(context%handle, int(n, c_int), rec, att, gate, up, down, an, pn, &
            c_loc(output_norm), int(size(output_norm), c_int), embedding_f16%handle, embedding_q8%handle, &
            output_f16%handle, output_q8%handle, int(max_context, c_int), norm_epsilon, self%handle)
        if (code /= FORTAI_HIP_OK) then
            self%handle = c_null_ptr
            self%context = c_null_ptr
        else
            self%context = context%handle
        end if
        call settle(code, context%handle, 'Qwen decoder creation', stat)
    end subroutine decoder_create

    subroutine decoder_destroy(self, stat)
        class(hip_qwen35_decoder_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle)) return
        code = fh_decoder_destroy(self%handle)
        self%handle = c_null_ptr
        self%context = c_null_ptr
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, 'HIP Qwen decoder destruction failed')
    end subroutine decoder_destroy

    subroutine decoder_reset(self, stat)
        class(hip_qwen35_decoder_t), intent(inout) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen decoder')
            return
        end if
        call settle(fh_decoder_reset(self%handle), self%context, 'Qwen decoder reset', stat)
    end subroutine decoder_reset

    ! One step; logits (vocab) and next_token (0-based greedy id) are returned.
    subroutine decoder_forward(self, token, position, logits, next_token, stat)
        class(hip_qwen35_decoder_t), intent(inout) :: self
        integer(c_int64_t), intent(in) :: token
        integer, intent(in) :: position
        real(c_float), contiguous, target, intent(out) :: logits(:)
        integer(c_int64_t), target, intent(out) :: next_token
        type(status_t), intent(out) :: stat

        call stat%clear()
        next_token = -1
        if (.not. live(self%handle) .or. token < 0 .or. position < 0 .or. size(logits) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen decoder step')
            return
        end if
        call settle(fh_decoder_forward(self%handle, token, int(position, c_int), c_loc(logits), &
            c_loc(next_token)), self%context, 'Qwen decoder step', stat)
    end subroutine decoder_forward

    ! Greedy decode of size(trace) tokens from (token, position), device resident.
    subroutine decoder_generate(self, token, position, trace, stat)
        class(hip_qwen35_decoder_t), intent(inout) :: self
        integer(c_int64_t), intent(in) :: token
        integer, intent(in) :: position
        integer(c_int64_t), contiguous, target, intent(out) :: trace(:)
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. token < 0 .or. position < 0 .or. size(trace) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen decoder generation')
            return
        end if
        call settle(fh_decoder_generate(self%handle, token, int(position, c_int), int(size(trace), c_int), &
            c_loc(trace)), self%context, 'Qwen decoder generation', stat)
    end subroutine decoder_generate

    ! The launches of one step as text lines "operation<TAB>kernel<TAB>batch"
    ! (new_line separated): the fields of the reference's plan_step_t
    ! (src/fortai_plan_ir.f90:7-11), for plan_ir_t%append.
    subroutine decoder_plan(self, text, stat)
        class(hip_qwen35_decoder_t), intent(in) :: self
        character(len=:), allocatable, intent(out) :: text
        type(status_t), intent(out) :: stat
        character(kind=c_char), allocatable, target :: buf(:)
        integer(c_size_t) :: need
        integer :: i
        integer(c_int) :: code

        call stat%clear()
        text = ''
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen decoder')
            return
        end if
        code = fh_decoder_plan(self%handle, c_null_ptr, 0_c_size_t, need)
        if (code /= FORTAI_HIP_OK .or. need < 1) then
            call settle(code, self%context, 'Qwen decoder plan', stat)
            return
        end if
        allocate (buf(need))
        call settle(fh_decoder_plan(self%handle, c_loc(buf), need, need), self%context, 'Qwen decoder plan', stat)
        if (.not. stat%is_ok()) return
        allocate (character(len=int(need) - 1) :: text)
        do i = 1, int(need) - 1
            text(i:i) = buf(i)
        end do
    end subroutine decoder_plan

    ! ---- batched decoder (independent sequences, prompt prefill) ------------------

    ! As decoder_create, for `batch` sequences (1..8) that share the weights;
    ! the batch object holds every sequence's state and caches.
    subroutine batch_create(self, context, batch, recurrent, attention, ffn_gate, ffn_up, ffn_down, &
            attn_norm, post_norm, output_norm, embedding_f16, embedding_q8, output_f16, output_q8, &
            max_context, norm_epsilon, stat)
        class(hip_qwen35_batch_t), intent(inout) :: self
        class(hip_q8_context_t), intent(in) :: context
        integer, intent(in) :: batch
        type(hip_qwen35_recurrent_t), intent(in) :: recurrent(:)
        type(hip_qwen35_attention_t), intent(in) :: attention(:)
        type(hip_q8_weights_t), intent(in) :: ffn_gate(:), ffn_up(:), ffn_down(:)
        real(c_float), contiguous, target, intent(in) :: attn_norm(:, :), post_norm(:, :), output_norm(:)
        type(hip_f16_weights_t), intent(in) :: embedding_f16, output_f16
        type(hip_q8_weights_t), intent(in) :: embedding_q8, output_q8
        integer, intent(in) :: max_context
        real(c_float), intent(in) :: norm_epsilon
        type(status_t), intent(out) :: stat
        type(c_ptr), allocatable :: rec(:), att(:), gate(:), up(:), down(:), an(:), pn(:)
        integer :: n, i
        integer(c_int) :: code

        call stat%clear()
        n = size(ffn_gate)
        if (.not. live(context%handle) .or. n <= 0 .or. size(recurrent) /= n .or. size(attention) /= n .or. &
                size(ffn_up) /= n .or. size(ffn_down) /= n .or. size(attn_norm, 2) /= n .or. &
                size(post_norm, 2) /= n .or. size(attn_norm, 1) /= size(output_norm) .or. &
                size(post_norm, 1) /= size(output_norm) .or. max_context <= 0 .or. batch < 1 .or. batch > 8) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen batch arguments')
            return
        end if
        allocate (rec(n), att(n), gate(n), up(n), down(n), an(n), pn(n))
        do i = 1, n
            rec(i) = recurrent(i)%handle
            att(i) = attention(i)%handle
            gate(i) = ffn_gate(i)%handle
            up(i) = ffn_up(i)%handle
            down(i) = ffn_down(i)%handle
            an(i) = c_loc(attn_norm(1, i))
            pn(i) = c_loc(post_norm(1, i))
        end do
        if (live(self%handle)) call self%destroy(stat)
        code = fh_batch_create(context%handle, int(batch, c_int), int(n, c_int), rec, att, gate, up, down, an, &
            pn, c_loc(output_norm), int(size(output_norm), c_int), embedding_f16%handle, embedding_q8%handle, &
            output_f16%handle, output_q8%handle, int(max_context, c_int), norm_epsilon, self%handle)
        if (code /= FORTAI_HIP_OK) then
            self%handle = c_null_ptr
            self%context = c_null_ptr
            self%batch = 0
        else
            self%context = context%handle
            self%batch = batch
        end if
        call settle(code, context%handle, 'Qwen batch creation', stat)
    end subroutine batch_create

    subroutine batch_destroy(self, stat)
        class(hip_qwen35_batch_t), intent(inout) :: self
        type(status_t), intent(out) :: stat
        integer(c_int) :: code

        call stat%clear()
        if (.not. live(self%handle)) return
        code = fh_batch_destroy(self%handle)
        self%handle = c_null_ptr
        self%context = c_null_ptr
        self%batch = 0
        if (code /= FORTAI_HIP_OK) call stat%set(FORTAI_UNSUPPORTED, 'HIP Qwen batch destruction failed')
    end subroutine batch_destroy

    subroutine batch_reset(self, stat)
        class(hip_qwen35_batch_t), intent(inout) :: self
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen batch')
            return
        end if
        call settle(fh_batch_reset(self%handle), self%context, 'Qwen batch reset', stat)
    end subroutine batch_reset

    ! Prompt tokens(t, s) of every sequence from position 0 (after reset);
    ! next_tokens(s) is the greedy token after the prompt.
    subroutine batch_prefill(self, tokens, next_tokens, stat)
        class(hip_qwen35_batch_t), intent(inout) :: self
        integer(c_int64_t), contiguous, target, intent(in) :: tokens(:, :)
        integer(c_int64_t), contiguous, target, intent(out) :: next_tokens(:)
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. size(tokens, 2) /= self%batch .or. size(tokens, 1) <= 0 .or. &
                size(next_tokens) /= self%batch) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen batch prefill')
            return
        end if
        call settle(fh_batch_prefill(self%handle, c_loc(tokens), int(size(tokens, 1), c_int), c_loc(next_tokens), &
            c_null_ptr, c_null_ptr), self%context, 'Qwen batch prefill', stat)
    end subroutine batch_prefill

    ! Greedy decode of size(trace, 1) tokens per sequence from (tokens(s),
    ! positions(s)); trace(k, s), device resident in between.
    subroutine batch_generate(self, tokens, positions, trace, stat)
        class(hip_qwen35_batch_t), intent(inout) :: self
        integer(c_int64_t), contiguous, target, intent(in) :: tokens(:)
        integer(c_int), contiguous, target, intent(in) :: positions(:)
        integer(c_int64_t), contiguous, target, intent(out) :: trace(:, :)
        type(status_t), intent(out) :: stat

        call stat%clear()
        if (.not. live(self%handle) .or. size(tokens) /= self%batch .or. size(positions) /= self%batch .or. &
                size(trace, 2) /= self%batch .or. size(trace, 1) <= 0) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen batch generation')
            return
        end if
        call settle(fh_batch_generate(self%handle, c_loc(tokens), c_loc(positions), int(size(trace, 1), c_int), &
            c_loc(trace)), self%context, 'Qwen batch generation', stat)
    end subroutine batch_generate

    ! As decoder_plan, for one batched step (prefill false) or the last
    ! prompt prefill (prefill true).
    subroutine batch_plan(self, prefill, text, stat)
        class(hip_qwen35_batch_t), intent(in) :: self
        logical, intent(in) :: prefill
        character(len=:), allocatable, intent(out) :: text
        type(status_t), intent(out) :: stat
        character(kind=c_char), allocatable, target :: buf(:)
        integer(c_size_t) :: need
        integer(c_int) :: which
        integer :: i

        call stat%clear()
        text = ''
        if (.not. live(self%handle)) then
            call stat%set(FORTAI_INVALID, 'invalid HIP Qwen batch decoder')
            return
        end if
        which = 0_c_int
        if (prefill) which = 1_c_int
        call settle(fh_batch_plan(self%handle, which, c_null_ptr, 0_c_size_t, need), self%context, &
            'Qwen batch plan', stat)
        if (.not. stat%is_ok()) return
        if (need < 1) then
            call stat%set(FORTAI_INVALID, 'Qwen batch plan is empty')
            return
        end if
        allocate (buf(need))
        call settle(fh_batch_plan(self%handle, which, c_loc(buf), need, need), self%context, 'Qwen batch plan', stat)
        if (.not. stat%is_ok()) return
        allocate (character(len=int(need) - 1) :: text)
        do i = 1, int(need) - 1
            text(i:i) = buf(i)
        end do
    end subroutine batch_plan

end module fortai_backend_hip
