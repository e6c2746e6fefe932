function initstacks_burgers1d_b(n, nsteps)
    branch_stack = Vector{Int64}(undef, max(0, div(nsteps - 1, 1) + 1))
    u_stack = Vector{Float64}(undef, max(0, div(nsteps - 1, 1) + 1) * max(0, div(n - 1, 1) + 1))
    return (branch_stack, u_stack)
end

function burgers1d_b(loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n, nsteps, branch_stack, u_stack)
    cadvb = 0.0
    cdifb = 0.0
    tcb = 0.0
    ucb = 0.0
    cadv = 0.5 * dt / dx
    cdif = nu * dt / (dx * dx)
    tc = 0.0
    for i_t = 1:nsteps
        if tc < tend
            __idx_branch_stack_0 = (i_t - 1) + 1
            branch_stack[__idx_branch_stack_0] = 1
            for i_x = 1:n
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                uc = u[i_x]
                un[i_x] = uc - cadv * uc * (u[ip] - u[im]) + cdif * (u[ip] - 2.0 * uc + u[im])
            end
            for i_x2 = 1:n
                __idx_u_stack_1 = ((i_x2 - 1) + (i_t - 1) * (div(n - 1, 1) + 1)) + 1
                u_stack[__idx_u_stack_1] = u[i_x2]
                u[i_x2] = un[i_x2]
            end
            tc = tc + dt
        else
            __idx_branch_stack_0 = (i_t - 1) + 1
            branch_stack[__idx_branch_stack_0] = 0
        end
    end
    for i_k = 1:n
        loss[1] = loss[1] + u[i_k] ^ 2
    end
    for i_k = n:-1:1
        ub[i_k] = ub[i_k] + (2 * u[i_k]) * lossb[1]
    end
    for i_t = nsteps:-1:1
        __idx_branch_stack_0 = (i_t - 1) + 1
        __branch = branch_stack[__idx_branch_stack_0]
        if __branch == 1
            dtb = dtb + tcb
            for i_x2 = n:-1:1
                __idx_u_stack_1 = ((i_x2 - 1) + (i_t - 1) * (div(n - 1, 1) + 1)) + 1
                u[i_x2] = u_stack[__idx_u_stack_1]
                __oldb_1 = ub[i_x2]
                ub[i_x2] = 0.0
                unb[i_x2] = unb[i_x2] + __oldb_1
            end
            for i_x = n:-1:1
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                uc = u[i_x]
                __oldb_2 = unb[i_x]
                unb[i_x] = 0.0
                __cse_3 = u[ip] - u[im]
                __cse_4 = -__oldb_2
                ucb = ucb + __oldb_2
                cadvb = cadvb + (uc * __cse_3) * __cse_4
                ucb = ucb + (cadv * __cse_3) * __cse_4
                __cse_5 = cadv * uc
                ub[ip] = ub[ip] + __cse_5 * __cse_4
                ub[im] = ub[im] + -(__cse_5 * __cse_4)
                cdifb = cdifb + (u[ip] - 2.0 * uc + u[im]) * __oldb_2
                __cse_6 = cdif * __oldb_2
                ub[ip] = ub[ip] + __cse_6
                ucb = ucb + 2.0 * -__cse_6
                ub[im] = ub[im] + __cse_6
                __oldb_7 = ucb
                ucb = 0.0
                ub[i_x] = ub[i_x] + __oldb_7
            end
        end
    end
    __oldb_8 = cdifb
    cdifb = 0.0
    __cse_9 = dx * dx
    nub = nub + (dt / __cse_9) * __oldb_8
    dtb = dtb + (nu / __cse_9) * __oldb_8
    __cse_10 = -((nu * dt) / __cse_9 ^ 2) * __oldb_8
    dxb = dxb + dx * __cse_10
    dxb = dxb + dx * __cse_10
    __oldb_11 = cadvb
    cadvb = 0.0
    dtb = dtb + (0.5 / dx) * __oldb_11
    dxb = dxb + -((0.5 * dt) / dx ^ 2) * __oldb_11
    return (nub, dtb, dxb, tendb)
end

function burgers1d(loss, u, un, nu, dt, dx, tend, n, nsteps)
    cadv = 0.5 * dt / dx
    cdif = nu * dt / (dx * dx)
    tc = 0.0
    for i_t = 1:nsteps
        if tc < tend
            for i_x = 1:n
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                uc = u[i_x]
                un[i_x] = uc - cadv * uc * (u[ip] - u[im]) + cdif * (u[ip] - 2.0 * uc + u[im])
            end
            for i_x2 = 1:n
                u[i_x2] = un[i_x2]
            end
            tc = tc + dt
        end
    end
    for i_k = 1:n
        loss[1] = loss[1] + u[i_k] ^ 2
    end
    return nothing
end
