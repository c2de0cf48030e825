! ref_time.f90 -- timing driver for the compiled reference CPU path.
!
! TEST INFRASTRUCTURE ONLY (built by oracle/Makefile into oracle/_ref/ and
! oracle/_ref/fast/).  It is this repository's own program; it links the
! reference's unmodified modules and times model%forward + the greedy maxloc
! the way app/fortai_cpu_run.f90:50-64 does, but for STEPS steps starting at
! position START: the key/value caches below START hold zeros, which is the
! same work per step as a cache filled by decoding (the attention reads every
! position up to the current one either way).
!
! usage: ref_time MODEL.gguf TOKEN STEPS CONTEXT START
! prints: forward_seconds=<s>  last_token=<id>
program ref_time
    use, intrinsic :: iso_fortran_env, only: int64, real32, real64
    use fortai_qwen35_cpu, only: qwen35_cpu_model_t
    use fortai_status, only: status_t
    implicit none

    type(qwen35_cpu_model_t) :: model
    type(status_t) :: stat
    real(real32), allocatable :: logits(:)
    character(len=1024) :: model_path, argument
    integer(int64) :: token, steps, context, start, position, t0, t1, rate
    integer :: ios

    call get_command_argument(1, model_path)
    call get_command_argument(2, argument)
    read (argument, *, iostat=ios) token
    call get_command_argument(3, argument)
    read (argument, *, iostat=ios) steps
    call get_command_argument(4, argument)
    read (argument, *, iostat=ios) context
    call get_command_argument(5, argument)
    read (argument, *, iostat=ios) start
    if (len_trim(model_path) == 0 .or. steps <= 0 .or. start < 0 .or. start + steps > context) then
        print '(a)', 'usage: ref_time MODEL.gguf TOKEN STEPS CONTEXT START'
        error stop 2
    end if
    call model%open(trim(model_path), context, stat)
    if (.not. stat%is_ok()) then
        print '(a)', 'open failed: '//stat%message
        error stop 1
    end if
    allocate (logits(model%vocabulary_size))
    call system_clock(t0, rate)
    do position = start, start + steps - 1_int64
        call model%forward(token, position, logits, stat)
        if (.not. stat%is_ok()) then
            print '(a)', 'forward failed: '//stat%message
            error stop 1
        end if
        token = int(maxloc(logits, dim=1) - 1, int64)
    end do
    call system_clock(t1)
    print '(a,es16.8)', 'forward_seconds=', real(t1 - t0, real64) / real(rate, real64)
    print '(a,i0)', 'last_token=', token
    call model%close()
end program ref_time
