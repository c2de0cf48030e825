! hip_plan_record.f90 -- records the HIP decoders' launch plans into the
! reference's PlanIR, from Fortran.
!
! TEST INFRASTRUCTURE ONLY (built by oracle/Makefile target ref-hip).  The
! reference's unmodified model (src/models/qwen35/fortai_qwen35_cpu.f90) is
! opened and moved to the device with its own enable_cuda(0)
! (fortai_qwen35_cpu.f90:287-384), which in this build creates every layer
! and weight through libfortai_hip.so.  Over those objects the program then
! creates the fused decoder (hip_qwen35_decoder_t) and a two-sequence batch
! decoder, decodes STEPS greedy tokens with each, and records each step's
! launches as plan_ir_t steps (src/fortai_plan_ir.f90:7-21) through
! fortai_hip_plan.  It prints
!   trace <ids>                  the fused decoder's greedy ids
!   batch trace <ids>            sequence 1 of the batch decoder
!   decoder plan <n>             then one "step <i> <operation> | <kernel> | <batch>" line each
!   batch plan <n>               the same for the batched step
! and "hip plan record ok" after plan_ir_t%validate succeeded for both.
!
! usage: hip_plan_record MODEL.gguf TOKEN STEPS CONTEXT
program hip_plan_record
    use, intrinsic :: iso_c_binding, only: c_float, c_int, c_int64_t
    use, intrinsic :: iso_fortran_env, only: int64
    use fortai_status, only: status_t
    use fortai_plan_ir, only: plan_ir_t
    use fortai_qwen35_cpu, only: qwen35_cpu_model_t
    use fortai_backend_hip, only: hip_qwen35_decoder_t, hip_qwen35_batch_t, hip_qwen35_recurrent_t, &
        hip_qwen35_attention_t, hip_q8_weights_t, hip_f16_weights_t
    use fortai_hip_plan, only: hip_decoder_plan_ir, hip_batch_plan_ir
    implicit none

    type(qwen35_cpu_model_t) :: model
    type(status_t) :: stat
    type(hip_qwen35_decoder_t) :: decoder
    type(hip_qwen35_batch_t) :: batch
    type(plan_ir_t) :: plan
    type(hip_qwen35_recurrent_t), allocatable :: rec(:)
    type(hip_qwen35_attention_t), allocatable :: att(:)
    type(hip_q8_weights_t), allocatable :: gate(:), up(:), down(:)
    type(hip_f16_weights_t) :: no_f16
    real(c_float), allocatable :: attn_norm(:, :), post_norm(:, :), output_norm(:)
    integer(c_int64_t), allocatable :: trace(:), btrace(:, :)
    integer(c_int64_t) :: token
    integer(int64) :: context
    integer :: steps, n, hidden, i, ios
    character(len=1024) :: model_path, argument

    call get_command_argument(1, model_path)
    call get_command_argument(2, argument)
    read (argument, *, iostat=ios) token
    call get_command_argument(3, argument)
    read (argument, *, iostat=ios) steps
    call get_command_argument(4, argument)
    read (argument, *, iostat=ios) context
    if (len_trim(model_path) == 0 .or. steps <= 0 .or. context <= 0) then
        print '(a)', 'usage: hip_plan_record MODEL.gguf TOKEN STEPS CONTEXT'
        error stop 2
    end if

    call model%open(trim(model_path), context, stat)
    call need('open')
    call model%enable_cuda(0, stat)
    call need('enable_cuda')

    n = size(model%layers)
    hidden = model%hidden_size
    allocate (rec(n), att(n), gate(n), up(n), down(n), attn_norm(hidden, n), post_norm(hidden, n))
    allocate (output_norm(hidden))
    do i = 1, n
        rec(i) = model%layers(i)%cuda_recurrent
        att(i) = model%layers(i)%cuda_attention
        gate(i) = model%cuda_weights(model%layers(i)%ffn_gate)
        up(i) = model%cuda_weights(model%layers(i)%ffn_up)
        down(i) = model%cuda_weights(model%layers(i)%ffn_down)
        call host_values(model%layers(i)%attn_norm, attn_norm(:, i))
        call host_values(model%layers(i)%post_norm, post_norm(:, i))
    end do
    call host_values(model%output_norm, output_norm)

    ! the fused decoder over the model's own device layers and weights
    call decoder%create(model%cuda, rec, att, gate, up, down, attn_norm, post_norm, output_norm, no_f16, &
        model%cuda_weights(model%token_embedding), no_f16, model%cuda_weights(model%output), int(context), &
        model%norm_epsilon, stat)
    call need('decoder create')
    allocate (trace(steps))
    call decoder%generate(token, 0, trace, stat)
    call need('decoder generate')
    print '(a,*(1x,i0))', 'trace', trace
    call hip_decoder_plan_ir(decoder, plan, stat)
    call need('decoder PlanIR')
    call print_plan('decoder plan')

    ! two sequences of the batch decoder, both from the same token
    call batch%create(model%cuda, 2, rec, att, gate, up, down, attn_norm, post_norm, output_norm, no_f16, &
        model%cuda_weights(model%token_embedding), no_f16, model%cuda_weights(model%output), int(context), &
        model%norm_epsilon, stat)
    call need('batch create')
    allocate (btrace(steps, 2))
    call batch%generate([token, token], [0_c_int, 0_c_int], btrace, stat)
    call need('batch generate')
    print '(a,*(1x,i0))', 'batch trace', btrace(:, 1)
    call hip_batch_plan_ir(batch, .false., plan, stat)
    call need('batch PlanIR')
    call print_plan('batch plan')

    call batch%destroy(stat)
    call decoder%destroy(stat)
    call model%close()
    print '(a)', 'hip plan record ok'

contains

    subroutine host_values(tensor, values)
        integer, intent(in) :: tensor
        real(c_float), intent(out) :: values(:)
        integer :: j
        do j = 1, size(values)
            values(j) = model%file%tensors(tensor)%value(int(j, int64))
        end do
    end subroutine host_values

    subroutine print_plan(title)
        character(len=*), intent(in) :: title
        integer :: s
        print '(a,1x,i0)', title, plan%count()
        do s = 1, plan%count()
            print '(a,i0,a)', 'step ', s, ' ' // plan%steps(s)%operation // ' | ' // plan%steps(s)%kernel // ' | ' // &
                trim(itoa(plan%steps(s)%batch_size))
        end do
    end subroutine print_plan

    function itoa(v) result(text)
        integer, intent(in) :: v
        character(len=16) :: text
        write (text, '(i0)') v
    end function itoa

    subroutine need(what)
        character(len=*), intent(in) :: what
        if (.not. stat%is_ok()) then
            print '(a)', 'FAILED: ' // what // ': ' // stat%message
            error stop 1
        end if
    end subroutine need

end program hip_plan_record
