! ref_dump.f90 -- golden-vector driver for the compiled reference CPU path.
!
! TEST INFRASTRUCTURE ONLY (built by oracle/Makefile into oracle/_ref/).  It is
! this repository's own program; it links the reference's unmodified modules
! (fortai_qwen35_cpu, fortai_status), compiled from /root/reference, and calls
! their public API the way app/fortai_cpu_run.f90:40-64 does, then writes the
! raw results the parity tests need:
!   <out>/logits.f32   [steps][vocab] logits of every step
!   <out>/tokens.i64   [steps] greedy ids (maxloc - 1, app/fortai_cpu_run.f90:58-61)
!   <out>/layer<L>.k.f32 / .v.f32   key/value cache of attention layer L after the run
!   <out>/layer<L>.gdn.f32 / .conv.f32   GDN and conv state of recurrent layer L
!
! usage: ref_dump MODEL.gguf TOKEN STEPS CONTEXT OUTDIR [DUMP_STATE(0|1)] [DEVICE(0|1)]
!
! DEVICE=1 calls the model's enable_cuda(0) (fortai_qwen35_cpu.f90:287-384)
! after open.  In the ref_dump_hip build the reference model is compiled
! against fortai_amd/fortran/fortai_backend_cuda_on_hip.f90, so that call
! moves its device pipeline onto libfortai_hip.so; the state dump then reads
! the CPU-side buffers, which the device pipeline does not update.
program ref_dump
    use, intrinsic :: iso_fortran_env, only: int64, real32
    use fortai_qwen35_cpu, only: qwen35_cpu_model_t
    use fortai_status, only: status_t
    implicit none

    type(qwen35_cpu_model_t) :: model
    type(status_t) :: stat
    real(real32), allocatable :: logits(:)
    character(len=1024) :: model_path, out_dir, argument
    integer(int64) :: token, steps, context, position
    integer(int64), allocatable :: trace(:)
    integer :: unit_logits, unit_tokens, ios, dump_state, layer, device
    character(len=32) :: tag

    call get_command_argument(1, model_path)
    call get_command_argument(2, argument)
    read (argument, *, iostat=ios) token
    call get_command_argument(3, argument)
    read (argument, *, iostat=ios) steps
    call get_command_argument(4, argument)
    read (argument, *, iostat=ios) context
    call get_command_argument(5, out_dir)
    dump_state = 0
    call get_command_argument(6, argument)
    if (len_trim(argument) > 0) read (argument, *, iostat=ios) dump_state
    device = 0
    call get_command_argument(7, argument)
    if (len_trim(argument) > 0) read (argument, *, iostat=ios) device
    if (len_trim(model_path) == 0 .or. len_trim(out_dir) == 0 .or. steps <= 0) then
        print '(a)', 'usage: ref_dump MODEL.gguf TOKEN STEPS CONTEXT OUTDIR [DUMP_STATE]'
        error stop 2
    end if

    call model%open(trim(model_path), context, stat)
    if (.not. stat%is_ok()) then
        print '(a)', 'open failed: '//stat%message
        error stop 1
    end if
    if (device /= 0) then
        call model%enable_cuda(0, stat)
        if (.not. stat%is_ok()) then
            print '(a)', 'enable device failed: '//stat%message
            error stop 1
        end if
    end if
    allocate (logits(model%vocabulary_size), trace(steps))
    open (newunit=unit_logits, file=trim(out_dir)//'/logits.f32', access='stream', &
        form='unformatted', status='replace')
    do position = 0_int64, steps - 1_int64
        call model%forward(token, position, logits, stat)
        if (.not. stat%is_ok()) then
            print '(a)', 'forward failed: '//stat%message
            error stop 1
        end if
        write (unit_logits) logits
        token = int(maxloc(logits, dim=1) - 1, int64)
        trace(position + 1) = token
        print '(a,i0,a,i0)', 'token[', position, ']=', token
    end do
    close (unit_logits)
    open (newunit=unit_tokens, file=trim(out_dir)//'/tokens.i64', access='stream', &
        form='unformatted', status='replace')
    write (unit_tokens) trace
    close (unit_tokens)

    if (dump_state /= 0) then
        do layer = 1, size(model%layers)
            write (tag, '(a,i0)') '/layer', layer - 1
            if (allocated(model%layers(layer)%key_cache)) then
                call dump(trim(out_dir)//trim(tag)//'.k.f32', model%layers(layer)%key_cache)
                call dump(trim(out_dir)//trim(tag)//'.v.f32', model%layers(layer)%value_cache)
            end if
            if (allocated(model%layers(layer)%gdn_state)) then
                call dump(trim(out_dir)//trim(tag)//'.gdn.f32', model%layers(layer)%gdn_state)
                call dump(trim(out_dir)//trim(tag)//'.conv.f32', model%layers(layer)%conv_state)
            end if
        end do
    end if
    call model%close()

contains

    subroutine dump(path, values)
        character(len=*), intent(in) :: path
        real(real32), intent(in) :: values(:)
        integer :: u
        open (newunit=u, file=path, access='stream', form='unformatted', status='replace')
        write (u) values
        close (u)
    end subroutine dump

end program ref_dump
